// gsr_optim.hip — the trainer's optimizer step: Adam over the six parameter
// groups (gaussian_splatting/utils/optim.py:12-31 of kmurungi/custom-3dgs-cuda:
// torch.optim.Adam, eps 1e-15, default betas) with the trainer's clamps of the
// updated parameters fused in (scripts/train.py:171-176: opacity logits;
// utils/adc.py:90-93: log-scales).  One launch covers up to kAdamMaxTensors
// tensors; each work-group takes a 4096-element chunk of one of them and
// streams parameter, gradient and both moments through registers in 16-byte
// loads: 16 B in and 12 B out per element, nothing else.
//
// Arithmetic per element, fp32, as torch.optim.Adam's default path evaluates it
// on the device (torch/optim/adam.py, _multi_tensor_adam: the foreach kernels,
// whose device code forms these fused multiply-adds), every scalar rounded to
// fp32 once from the host's double as torch does with a Python scalar:
//   m = fma(1 - b1, g - m, m)                          (_foreach_lerp_)
//   v = fma(1 - b2, g g, v b2)                         (_foreach_mul_, _foreach_addcmul_)
//   p = fma(-step_size, m / (sqrt(v) / sqrt(bc2) + eps), p)   (_foreach_addcdiv_)
//   p = clamp(p, lo, hi), NaN kept                     (clamp_)
// with correctly rounded sqrt (sqrt_rn, gsr_common.h) and division (__fdiv_rn: the
// div_scale / div_fmas / div_fixup sequence) and no other contraction (the
// library is built with -ffp-contract=off).  The trainer runs Adam on the
// device, so this is the rounding it trains with; torch's CPU single-tensor
// path forms v = fma((1 - b2) g, g, v b2) and p + (-step_size m) / d instead.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "gsr_common.h"
#include "gsr_internal.h"

namespace gsr {

namespace {

constexpr int kAdamThreads = 256;
constexpr int kAdamVec = 4;  // float4 per load
constexpr int kAdamChunk = kAdamThreads * kAdamVec * 4;  // elements per work-group

struct AdamScalars {
    float w1, b2, w2, bc2s, neg_step, eps, lo, hi;
};

__device__ __forceinline__ void adam_update(float& p, float g, float& m, float& v,
                                            const AdamScalars& s) {
    m = __builtin_fmaf(s.w1, g - m, m);
    v = __builtin_fmaf(s.w2, g * g, v * s.b2);
    const float d = __fdiv_rn(sqrt_rn(v), s.bc2s) + s.eps;
    float x = __builtin_fmaf(s.neg_step, __fdiv_rn(m, d), p);
    x = (x < s.lo) ? s.lo : x;
    x = (x > s.hi) ? s.hi : x;
    p = x;
}

struct AdamBatch {
    AdamTensor t[kAdamMaxTensors];
    AdamScalars s[kAdamMaxTensors];
    uint32_t chunk0[kAdamMaxTensors + 1];
    int count;
};

__global__ __launch_bounds__(kAdamThreads) void adam_kernel(AdamBatch b) {
    // the tensor of this work-group's chunk (uniform: a scalar loop)
    int i = 0;
    while (i + 1 < b.count && blockIdx.x >= b.chunk0[i + 1]) ++i;
    const AdamTensor t = b.t[i];
    const AdamScalars s = b.s[i];
    const uint64_t base = (uint64_t)(blockIdx.x - b.chunk0[i]) * kAdamChunk;
    const uint64_t n = t.numel;
    const bool vec = ((reinterpret_cast<uintptr_t>(t.param) | reinterpret_cast<uintptr_t>(t.grad) |
                       reinterpret_cast<uintptr_t>(t.exp_avg) |
                       reinterpret_cast<uintptr_t>(t.exp_avg_sq)) & 15) == 0;
#pragma unroll
    for (int k = 0; k < kAdamChunk / (kAdamThreads * kAdamVec); ++k) {
        const uint64_t e = base + ((uint64_t)k * kAdamThreads + threadIdx.x) * kAdamVec;
        if (vec && e + kAdamVec <= n) {
            // each element is touched once: non-temporal (streaming) loads and
            // stores (1.54 to 1.46 ms at 5M Gaussians, 67% to 71% of HBM)
            f32x4 p = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(t.param + e));
            const f32x4 g = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(t.grad + e));
            f32x4 m = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(t.exp_avg + e));
            f32x4 v =
                __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(t.exp_avg_sq + e));
#pragma unroll
            for (int c = 0; c < kAdamVec; ++c) {
                float pc = p[c], mc = m[c], vc = v[c];
                adam_update(pc, g[c], mc, vc, s);
                p[c] = pc;
                m[c] = mc;
                v[c] = vc;
            }
            __builtin_nontemporal_store(p, reinterpret_cast<f32x4*>(t.param + e));
            __builtin_nontemporal_store(m, reinterpret_cast<f32x4*>(t.exp_avg + e));
            __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(t.exp_avg_sq + e));
        } else {
            for (uint64_t j = e; j < e + kAdamVec && j < n; ++j) {
                float p = t.param[j], m = t.exp_avg[j], v = t.exp_avg_sq[j];
                adam_update(p, t.grad[j], m, v, s);
                t.param[j] = p;
                t.exp_avg[j] = m;
                t.exp_avg_sq[j] = v;
            }
        }
    }
}

}  // namespace

hipError_t launch_adam(int count, const AdamTensor* tensors, const AdamHostScalars* hs,
                       hipStream_t st) {
    for (int first = 0; first < count; first += kAdamMaxTensors) {
        AdamBatch b{};
        b.count = std::min(kAdamMaxTensors, count - first);
        uint64_t chunks = 0;
        for (int i = 0; i < b.count; ++i) {
            const AdamTensor& t = tensors[first + i];
            const AdamHostScalars& h = hs[first + i];
            b.t[i] = t;
            b.s[i] = AdamScalars{h.w1, h.b2, h.w2, h.bc2s, h.neg_step, h.eps, h.lo, h.hi};
            b.chunk0[i] = (uint32_t)chunks;
            chunks += (t.numel + kAdamChunk - 1) / kAdamChunk;
        }
        b.chunk0[b.count] = (uint32_t)chunks;
        if (chunks == 0) continue;
        if (chunks > 0x7fffffffull) return hipErrorInvalidValue;
        hipLaunchKernelGGL(adam_kernel, dim3((unsigned)chunks), dim3(kAdamThreads), 0, st, b);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace gsr
