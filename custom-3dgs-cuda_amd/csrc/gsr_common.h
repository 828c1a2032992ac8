// gsr_common.h — device helpers shared by the rasterizer kernels (gfx950, wave64).
//
// Every file in this library is compiled with -ffp-contract=off: the fp32
// forward math keeps the reference's operation order (one rounding per
// multiply and add), so projected means, covariances, colours and the blend's
// transmittance sequence are bit-identical to the CPU restatement.  The only
// fused multiply-adds are the explicit fmaf calls below.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gsr {

constexpr int kTileSize = 16;             // 16x16 pixel tiles (rasterize.cu:301)
constexpr int kTilePixels = 256;
constexpr int kWave = 64;                 // CDNA wavefront width
constexpr float kNearZ = 0.2f;            // projection.cu:47
constexpr float kAlphaMax = 0.99f;        // rasterize.cu:255
constexpr float kAlphaMin = 1.0f / 255.0f;  // rasterize.cu:256
constexpr float kTransmittanceMin = 1e-4f;  // rasterize.cu:265

// exp(x) in fp32: Cody–Waite reduction with fdlibm's split of ln2
// (0x3f317200 + 0x35bfbe8e), then a degree-6 polynomial for e^r on
// [-ln2/2, ln2/2] from a weighted least-squares fit on Chebyshev nodes
// (csrc/gen_exp_poly.py), Horner with fmaf, scaled by 2^k with ldexp.
// Faithfully rounded (max 0.955 ulp over [-87.34, 88.72]); results below
// FLT_MIN are flushed to +0.  Host and device evaluate the same IEEE
// operations, so their results agree bit for bit.
__device__ __forceinline__ float exp_gs(float x) {
    if (x > 88.72283935546875f) return __builtin_inff();
    if (!(x >= -87.33654022216796875f)) return (x != x) ? x : 0.0f;
    const float k = __builtin_rintf(x * 1.44269502162933349609375f);
    float r = __builtin_fmaf(-k, 0.693145751953125f, x);
    r = __builtin_fmaf(-k, 1.428606765330187045e-06f, r);
    float p = 0.0013766406336799264f;
    p = __builtin_fmaf(p, r, 0.00837041437625885f);
    p = __builtin_fmaf(p, r, 0.041669245809316635f);
    p = __builtin_fmaf(p, r, 0.16666485369205475f);
    p = __builtin_fmaf(p, r, 0.49999988079071045f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)k);
}

// Saturating float -> int32 with NaN -> 0 (the GPU conversion the reference's
// (int)floorf / (int)ceilf casts rely on, rasterize.cu:38-41), written out
// so no out-of-range cast is left to the compiler.
__device__ __forceinline__ int f2i_sat(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return 2147483647;
    if (x <= -2147483648.0f) return (-2147483647 - 1);
    return (int)x;
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

// Lanes strictly below this one.
__device__ __forceinline__ uint64_t lanemask_lt() {
    const int l = lane_id();
    return (l == 0) ? 0ull : (~0ull >> (64 - l));
}

__device__ __forceinline__ int popc64(uint64_t m) { return __builtin_popcountll(m); }

// Sum over the 64 lanes of a wave (result valid in every lane).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        uint32_t o = (uint32_t)__shfl_xor((int)v, off, kWave);
        v = v > o ? v : o;
    }
    return v;
}

// Inclusive prefix sum over the wave (u32).
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
    const int l = lane_id();
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        uint32_t o = (uint32_t)__shfl_up((int)v, off, kWave);
        if (l >= off) v += o;
    }
    return v;
}

// Device-coherent (agent scope) accesses for decoupled look-back status
// words: every wave on every XCD sees the latest value.
__device__ __forceinline__ uint64_t load_agent(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Look-back status word: flag in the top 2 bits, value in the low 62.
constexpr uint64_t kFlagAggregate = 1ull << 62;
constexpr uint64_t kFlagInclusive = 2ull << 62;
constexpr uint64_t kValueMask = (1ull << 62) - 1;
// Bound on look-back spins; a kernel that reaches it records an error and
// exits instead of waiting forever.
constexpr uint32_t kSpinLimit = 1u << 22;

// Per-Gaussian blend record (48 B), built once per frame from the
// rasterize inputs: (mean.x, mean.y, conic.x, 2*conic.y), (conic.z,
// opacity, r, g), (b, conic.y, -, -).  2*conic.y is an exact scaling of
// the reference's conic.y, so ((2*cy)*dx)*dy is the same product it forms.
struct __align__(16) BlendRec {
    float4 a;
    float4 b;
    float4 c;
};

}  // namespace gsr
