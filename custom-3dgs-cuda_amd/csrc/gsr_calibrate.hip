// gsr_calibrate.hip — VALU issue-rate calibration kernels (measurement
// support; no counterpart in the reference).
//
// Each kernel runs 8 independent dependency chains per lane of one
// instruction kind, 256-thread work-groups, 16 per CU.  Under rocprofv3 the
// issue counters of these kernels (SQ_INSTS_VALU, SQ_ACTIVE_INST_VALU,
// SQ_ACTIVE_INST_VALU2, GRBM_GUI_ACTIVE) show what fraction of the SIMDs'
// VALU issue cycles a kernel made only of that instruction reaches: the
// practical ceiling against which the blends' issue utilisation is read.
#include "gsr_internal.h"
#include "gsr_common.h"

namespace gsr {

namespace {

constexpr int kCalibThreads = 256;

template <int kKind>
__global__ __launch_bounds__(kCalibThreads) void calibrate_valu_kernel(float* __restrict__ out,
                                                                        int iters, float a,
                                                                        float b) {
    float v[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] = (float)threadIdx.x * 1e-3f + (float)c;
    for (int i = 0; i < iters; ++i) {
        if constexpr (kKind == 3) {
            // permlane swaps: four 32-lane and four 16-lane swaps per step
#pragma unroll
            for (int c = 0; c < 8; c += 2) {
                const auto r = __builtin_amdgcn_permlane32_swap(
                    __float_as_uint(v[c]), __float_as_uint(v[c + 1]), false, false);
                v[c] = __uint_as_float(r[0]);
                v[c + 1] = __uint_as_float(r[1]);
            }
#pragma unroll
            for (int c = 0; c < 8; c += 2) {
                const auto r = __builtin_amdgcn_permlane16_swap(
                    __float_as_uint(v[c]), __float_as_uint(v[c + 1]), false, false);
                v[c] = __uint_as_float(r[0]);
                v[c + 1] = __uint_as_float(r[1]);
            }
        } else {
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                if constexpr (kKind == 0) v[c] = v[c] + a;
                if constexpr (kKind == 1) v[c] = __builtin_fmaf(v[c], a, b);
                if constexpr (kKind == 2) v[c] = __builtin_amdgcn_exp2f(v[c]);
                if constexpr (kKind == 4) v[c] = v[c] + dpp_move<kDppRowRor8>(v[c]);
            }
        }
        a += 1e-7f;
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) s += v[c];
    out[(size_t)blockIdx.x * kCalibThreads + threadIdx.x] = s;
}

}  // namespace

int calibrate_valu_blocks() { return 256 * 16; }

hipError_t launch_calibrate_valu(int kind, int iters, float* out, hipStream_t st) {
    const dim3 grid(calibrate_valu_blocks()), block(kCalibThreads);
    switch (kind) {
        case 0: hipLaunchKernelGGL(calibrate_valu_kernel<0>, grid, block, 0, st, out, iters, 0.999f, 1e-3f); break;
        case 1: hipLaunchKernelGGL(calibrate_valu_kernel<1>, grid, block, 0, st, out, iters, 0.999f, 1e-3f); break;
        case 2: hipLaunchKernelGGL(calibrate_valu_kernel<2>, grid, block, 0, st, out, iters, 0.999f, 1e-3f); break;
        case 3: hipLaunchKernelGGL(calibrate_valu_kernel<3>, grid, block, 0, st, out, iters, 0.999f, 1e-3f); break;
        case 4: hipLaunchKernelGGL(calibrate_valu_kernel<4>, grid, block, 0, st, out, iters, 0.999f, 1e-3f); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gsr
