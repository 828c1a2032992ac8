// gsr_common.h — device helpers shared by the rasterizer kernels (gfx950, wave64).
//
// Every file in this library is compiled with -ffp-contract=off: the fp32
// forward math keeps the reference's operation order (one rounding per
// multiply and add), so projected means, covariances, colours and the blend's
// transmittance sequence are bit-identical to the CPU restatement.  The only
// fused multiply-adds in that math are explicit fmaf calls (the exp below,
// and the blend's power and colour sums, which the CPU restatement fuses in
// the same places).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gsr {

constexpr int kTileSize = 16;             // 16x16 pixel tiles (rasterize.cu:301)
constexpr int kTilePixels = 256;
constexpr int kWave = 64;                 // CDNA wavefront width

// Four floats as a native vector (the operand type of the non-temporal load
// and store builtins, which take no HIP float4).
typedef float f32x4 __attribute__((ext_vector_type(4)));
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
constexpr float kExpHi = 88.72283935546875f, kExpLo = -87.33654022216796875f;

// The reduction and polynomial for x in [kExpLo, kExpHi] (NaN stays NaN).
__device__ __forceinline__ float exp_core(float xc) {
    const float k = __builtin_rintf(xc * 1.44269502162933349609375f);
    float r = __builtin_fmaf(-k, 0.693145751953125f, xc);
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

// Branch-free: the polynomial runs on x clamped to the finite range (bit-identical
// for in-range x) and the out-of-range results are selected afterwards, so a
// wave never diverges inside exp.
__device__ __forceinline__ float exp_gs(float x) {
    const float e = exp_core(fminf(fmaxf(x, kExpLo), kExpHi));
    const float below = (x != x) ? x : 0.0f;
    return (x > kExpHi) ? __builtin_inff() : ((x >= kExpLo) ? e : below);
}

// exp_gs for the blends' G = exp(power): identical for x <= kExpHi and NaN.
// Larger x only occurs with power > 0, which both blends skip before G is
// used, so the upper clamp is left out (one compare and two selects).
__device__ __forceinline__ float exp_blend(float x) {
    const bool below = x < kExpLo;
    const float e = exp_core(below ? kExpLo : x);
    return below ? 0.0f : e;
}

// exp_blend with the polynomial run on x itself below kExpLo (its value there,
// finite or NaN, raises nothing on the GPU, and the select replaces it with
// 0): the same result for every x, one select fewer.  The forward step uses
// it; in the backward's exact re-evaluation the clamped form schedules better
// (the backward blend 215 against 221 us at 1080p).
__device__ __forceinline__ float exp_blend_noclamp(float x) {
    const bool below = x < kExpLo;
    const float e = exp_core(x);
    return below ? 0.0f : e;
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

// sqrt rounded to nearest, as the CPU's: the hardware square root (within
// 1 ulp; inputs below 2^-96 scaled by 2^32 first, the result by 2^-16), then
// a step to the neighbour on the side the exact residual x - s' s points to
// (the residual of a neighbour s' against s, one fused multiply-add each).
// Zero, infinity and NaN pass unchanged (their residuals are NaN or zero).
__device__ __forceinline__ float sqrt_rn(float x) {
    const bool small = x < 0x1p-96f;
    const float xs = small ? x * 0x1p+32f : x;
    float s = __builtin_amdgcn_sqrtf(xs);
    const float down = __int_as_float(__float_as_int(s) - 1);
    const float up = __int_as_float(__float_as_int(s) + 1);
    const float rd = __builtin_fmaf(-down, s, xs);
    const float ru = __builtin_fmaf(-up, s, xs);
    s = (rd <= 0.0f) ? down : s;
    s = (ru > 0.0f) ? up : s;
    return small ? s * 0x1p-16f : s;
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

// Lanes strictly below this one.
__device__ __forceinline__ uint64_t lanemask_lt() {
    const int l = lane_id();
    return (l == 0) ? 0ull : (~0ull >> (64 - l));
}

__device__ __forceinline__ int popc64(uint64_t m) { return __builtin_popcountll(m); }

// Adds one to LDS histogram bin d for every active lane.  A wave whose active
// lanes all have the same bin adds their count once: a bin hit by whole waves
// (a byte every key shares) would otherwise take 64 same-address atomics per
// instruction.
__device__ __forceinline__ void lds_hist_add(uint32_t* h, uint32_t d) {
    const uint64_t act = ballot(true);
    const uint32_t d0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)d);
    if (ballot(d != d0) == 0ull) {
        if ((act & lanemask_lt()) == 0ull) atomicAdd(&h[d0], (uint32_t)popc64(act));
    } else {
        atomicAdd(&h[d], 1u);
    }
}

// Sum over the 64 lanes of a wave (result valid in every lane).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// DPP lane moves within a 16-lane row (gfx9 encodings).
template <int Ctrl, int BankMask = 0xf>
__device__ __forceinline__ float dpp_move(float x, float old = 0.0f) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(x), Ctrl,
                                                      0xf, BankMask, false));
}
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppRowShl4 = 0x104;
constexpr int kDppRowShr4 = 0x114;
constexpr int kDppRowRor8 = 0x128;  // lane i <- lane i ^ 8 within the row

// lane i <- lane i ^ 4 within the row: two bank-masked moves (the first
// writes banks 1 and 3, the second banks 0 and 2, so no lane keeps the
// destination's old value).
__device__ __forceinline__ float lane_xor4(float x) {
    const float t = __int_as_float(
        __builtin_amdgcn_mov_dpp(__float_as_int(x), kDppRowShr4, 0xf, 0xa, false));
    return dpp_move<kDppRowShl4, 0x5>(x, t);
}

// a + b with their upper/lower 32-lane halves exchanged: lanes 0-31 get
// a[l] + a[l+32], lanes 32-63 get b[l-32] + b[l] (v_permlane32_swap, gfx950).
__device__ __forceinline__ float fold32(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Row-pair fold: rows 0,2 get a's (row0+row1, row2+row3), rows 1,3 get b's
// (v_permlane16_swap, gfx950).
__device__ __forceinline__ float fold16(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The backward's nine wave sums from six per-lane sums, for the blend layout
// where lanes l, l ^ 16, l ^ 32 and l ^ 48 hold the same pixel column (lane &
// 15, one dx per lane).  A transposed reduction: each level halves the live
// registers while doubling the lanes summed.  The 32- and 16-lane levels
// (permlane swaps) run on the six column-free sums only (S0, P2, P5, c0, c1,
// c2) and leave column totals; then dx S0, dx^2 S0 and dx P2 are formed per
// column and the 8-, 4-, 2- and 1-lane levels (row_ror, bank-masked row
// shifts, quad permutes) finish four registers.  ~27 VALU.  Value k's wave
// total ends in lane kColLane[k] of the result (and in the lanes of its quad).
// All 64 lanes must be active.
constexpr int kColS0 = 0, kColP1 = 1, kColQ1 = 2, kColP2 = 3, kColQ2 = 4, kColP5 = 5,
              kColC0 = 6, kColC1 = 7, kColC2 = 8;
constexpr int kColLane[9] = {0, 8, 4, 16, 24, 12, 32, 48, 44};

__device__ __forceinline__ float wave_reduce_columns(float s0, float p2, float p5, float c0,
                                                     float c1, float c2, float dx) {
    // lanes 0-31 (rows 0, 1) hold S0, P2, P5; lanes 32-63 (rows 2, 3) c0, c1, c2
    const float r0 = fold32(s0, c0);
    const float r1 = fold32(p2, c1);
    const float r2 = fold32(p5, c2);
    // column totals: a = (S0, P2, c0, c1) in rows 0-3, b = (P5, -, c2, -): b's
    // swap takes the first swap's spent register as its partner (its rows 1
    // and 3, summed into b's rows 1 and 3, reach no lane that holds a value)
    const auto s01 = __builtin_amdgcn_permlane16_swap(__float_as_uint(r0), __float_as_uint(r1),
                                                      false, false);
    const float a = __uint_as_float(s01[0]) + __uint_as_float(s01[1]);
    const auto s2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(r2), s01[0], false, false);
    const float b = __uint_as_float(s2[0]) + __uint_as_float(s2[1]);
    const float t1 = dx * a;   // row 0: dx S0, row 1: dx P2
    const float t2 = dx * t1;  // row 0: dx^2 S0
    const int l = lane_id();
    const bool b3 = (l & 8) != 0;
    const float u0 = (b3 ? t1 : a) + dpp_move<kDppRowRor8>(b3 ? a : t1);
    const float u1 = (b3 ? b : t2) + dpp_move<kDppRowRor8>(b3 ? t2 : b);
    const bool b2 = (l & 4) != 0;
    float w = (b2 ? u1 : u0) + lane_xor4(b2 ? u0 : u1);
    w = w + dpp_move<kDppQuadXor2>(w);
    w = w + dpp_move<kDppQuadXor1>(w);
    // formed here with every lane active, so the last level stays one DPP add
    // (a caller that only keeps the value in some lanes would otherwise have
    // the add sunk into its branch and the lane move split from it)
    asm volatile("" : "+v"(w));
    return w;
}

// Which of the nine values lane l holds after wave_reduce_columns (-1: none).
// Lane l with l & 3 == 0 holds, in row l >> 4, register (l >> 2) & 3 of the
// last levels: 0 a, 1 t2, 2 t1, 3 b.
__device__ __forceinline__ int columns_value_of_lane(int l) {
    if (l & 3) return -1;
    for (int k = 0; k < 9; ++k)
        if (kColLane[k] == l) return k;
    return -1;
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += (uint32_t)__shfl_xor((int)v, off, kWave);
    return v;
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, off, kWave);
        const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), off, kWave);
        v += ((uint64_t)hi << 32) | lo;
    }
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

// Inclusive prefix sums over the wave with DPP: row shifts by 1, 2, 4 and 8
// within each 16-lane row (lanes shifted in from outside the row read 0), then
// lane 15's row total broadcast to rows 1 and 3 and lane 31's to rows 2 and 3
// (gfx9 row_bcast).  Twelve VALU, no LDS.
template <int Ctrl, int RowMask>
__device__ __forceinline__ uint32_t dpp_or_zero(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, Ctrl, RowMask, 0xf, true);
}
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112,
              kDppRowShr8 = 0x118, kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;

__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
    v += dpp_or_zero<kDppRowShr1, 0xf>(v);
    v += dpp_or_zero<kDppRowShr2, 0xf>(v);
    v += dpp_or_zero<kDppRowShr4, 0xf>(v);
    v += dpp_or_zero<kDppRowShr8, 0xf>(v);
    v += dpp_or_zero<kDppRowBcast15, 0xa>(v);
    v += dpp_or_zero<kDppRowBcast31, 0xc>(v);
    return v;
}

__device__ __forceinline__ float wave_inclusive_scan_f(float v) {
    auto step = [](float x, uint32_t y) { return x + __uint_as_float(y); };
    v = step(v, dpp_or_zero<kDppRowShr1, 0xf>(__float_as_uint(v)));
    v = step(v, dpp_or_zero<kDppRowShr2, 0xf>(__float_as_uint(v)));
    v = step(v, dpp_or_zero<kDppRowShr4, 0xf>(__float_as_uint(v)));
    v = step(v, dpp_or_zero<kDppRowShr8, 0xf>(__float_as_uint(v)));
    v = step(v, dpp_or_zero<kDppRowBcast15, 0xa>(__float_as_uint(v)));
    v = step(v, dpp_or_zero<kDppRowBcast31, 0xc>(__float_as_uint(v)));
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
// rasterize inputs: (mean.x, mean.y, -conic.x/2, -conic.y), (-conic.z/2,
// opacity, r, g), (b, -conic.y/2, qthr, -).  The conic terms carry the
// power's -1/2 (exact scalings by powers of two), so the blend evaluates
// power = fma(c dy, dy, fma(b dx, dy, (a dx) dx)) without the final multiply;
// the conic itself is -2 times them, exactly.
// qthr bounds the quadratic form from above for any pixel that can reach
// alpha >= 1/255 (conservative; negative when the opacity alone rules every
// pixel out): the blends use it to skip entries for whole pixel regions
// without changing any per-pixel result.
struct __align__(16) BlendRec {
    float4 a;
    float4 b;
    float4 c;
};

// Threshold on q = d^T conic d above which o * exp(-q/2) < 1/255, so alpha
// stays below 1/255 (rasterize.cu:256): 2 ln(255 o), computed in double and
// raised by 1e-5 relative + 1e-4 to cover exp_gs (<= 1 ulp), the o * G
// product and the rounding of this threshold.  NaN for a NaN opacity, which
// then disables every cull.
__device__ __forceinline__ float alpha_q_threshold(float o) {
    const double t = 2.0 * log(255.0 * (double)o);
    return (float)(t + 1e-5 * fabs(t) + 1e-4);
}

// Conic = cov^-1 with 1/det first (rasterize.cu:224-232), packed with mean,
// opacity and colour so the blend loads one 48 B record per list entry.
__device__ __forceinline__ BlendRec blend_record(float mx, float my, float a, float b, float c,
                                                 float opacity, float r, float g, float bl) {
    const float det = a * c - b * b;
    const float det_inv = (det > 0.0f) ? (1.0f / det) : 0.0f;
    const float cx = c * det_inv, cy = -b * det_inv, cz = a * det_inv;
    BlendRec rec;
    rec.a = make_float4(mx, my, -0.5f * cx, -cy);
    rec.b = make_float4(-0.5f * cz, opacity, r, g);
    rec.c = make_float4(bl, -0.5f * cy, alpha_q_threshold(opacity), 0.0f);
    return rec;
}

}  // namespace gsr
