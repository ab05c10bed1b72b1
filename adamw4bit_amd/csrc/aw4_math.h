// Scalar arithmetic, cross-lane primitives and the counter-based generator of the fused step.
//
// ATen's fp32 multiply, add, division, reciprocal and fused multiply-add (lerp) are
// correctly rounded, and so are the routines here that stand in for them wherever a
// result feeds a code or a block scale.  ATen's CPU square root comes from a vector
// math library and is only faithful (within one ulp of the correctly rounded value,
// and host dependent), so the square roots here are the hardware's faithful one:
// values downstream of a square root (the parameter update, update-SR preconditioners)
// agree with the reference to about one ulp, as the reference agrees with itself
// across hosts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aw4 {

// Global-memory pointers.  Device addresses read from a launch table are generic (flat)
// pointers to the compiler; a flat access also counts against the LDS wait counter, so
// every wait for an LDS table read would wait for the outstanding global loads and
// stores too.  Casting to address space 1 gives global_* instructions (scalar base +
// 32-bit lane offset) that leave LDS waits independent of HBM traffic.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef double f64x2 __attribute__((ext_vector_type(2)));

template <class T>
using gptr = __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ gptr<T> gaddr(uint64_t a) { return (gptr<T>)a; }

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

// ATen's clamp_min / clamp propagate NaN.
__device__ __forceinline__ float clamp_min_nan(float x, float lo) { return x < lo ? lo : x; }
__device__ __forceinline__ float clamp01_nan(float x) { return x < 0.0f ? 0.0f : (x > 1.0f ? 1.0f : x); }

// RN(v / s) from y = RN(1 / s): one FMA correction of RN(v * y) (Markstein).  Exact
// for normal quotients; a subnormal quotient may differ from RN(v / s) by a few
// subnormal ulps, which no code or scale of the codec can observe (see encode_block).
__device__ __forceinline__ float div_by_rcp(float v, float s, float y) {
    const float q = v * y;
    const float r = __builtin_fmaf(-q, s, v);
    return __builtin_fmaf(r, y, q);
}

// RN(n / d): hardware reciprocal (<= 1 ulp), one Newton step, one Markstein
// correction of the quotient, and the hardware fix-up for zero, infinite and NaN
// operands.  Correctly rounded for normal quotients (checked against IEEE
// division on 3e8 operand pairs with reciprocal seeds perturbed by +-1 ulp).
__device__ __forceinline__ float div_cr(float n, float d) {
    const float y0 = __builtin_amdgcn_rcpf(d);
    const float e0 = __builtin_fmaf(-d, y0, 1.0f);
    const float y1 = __builtin_fmaf(e0, y0, y0);
    const float q0 = n * y1;
    const float r0 = __builtin_fmaf(-d, q0, n);
    const float q1 = __builtin_fmaf(r0, y1, q0);
    return __builtin_amdgcn_div_fixupf(q1, d, n);
}

// RN(sqrt(x)) for x >= -0: hardware square root (<= 1 ulp) corrected by the sign of
// the residuals x - (y -+ ulp) * y; inputs below 2^-96 are scaled by 2^32 so the
// residual products stay normal.  +-0, +inf and NaN pass through unchanged.
__device__ __forceinline__ float sqrt_cr(float x) {
    const bool tiny = x < 0x1p-96f;
    const float xs = tiny ? x * 0x1p+32f : x;
    float y = __builtin_amdgcn_sqrtf(xs);
    const float ydn = u2f(f2u(y) - 1u);
    const float yup = u2f(f2u(y) + 1u);
    const float rdn = __builtin_fmaf(-ydn, y, xs);
    const float rup = __builtin_fmaf(-yup, y, xs);
    y = rdn <= 0.0f ? ydn : y;
    y = rup > 0.0f ? yup : y;
    return tiny ? y * 0x1p-16f : y;
}

// Faithful sqrt (v_sqrt_f32, <= 1 ulp), the precision class of ATen's CPU sqrt.
__device__ __forceinline__ float sqrt_faithful(float x) { return __builtin_amdgcn_sqrtf(x); }

// Reciprocal within one ulp: hardware estimate refined by one Newton step.
__device__ __forceinline__ float rcp_faithful(float t) {
    const float y0 = __builtin_amdgcn_rcpf(t);
    const float e0 = __builtin_fmaf(-t, y0, 1.0f);
    return __builtin_fmaf(e0, y0, y0);
}

// bf16 round-to-nearest-even (c10::BFloat16), NaN kept quiet, by v_cvt_pk_bf16_f32: on MI355X it
// gives the bits of the integer rule (u + 0x7fff + ((u >> 16) & 1)) >> 16, and (u >> 16) | 0x40 for
// a NaN, for every one of the 2^32 fp32 inputs, subnormals included.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
// two values, packed (low half: a)
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}
__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return u2f(h << 16); }
// IEEE binary16, round-to-nearest-even (v_cvt_f16_f32), subnormals kept.
__device__ __forceinline__ uint32_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// ---------------------------------------------------------------------------
// Cross-lane primitives (DPP within the 8 lanes of a block)
// ---------------------------------------------------------------------------

template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, 0xF, 0xF, false);
}
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}
constexpr int kQuadXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kHalfRowMirror = 0x141;  // lane i <- lane 7 - i within 8 lanes
constexpr int kRowShl1 = 0x101, kRowShl2 = 0x102, kRowShl4 = 0x104, kRowShl6 = 0x106;  // lane i <- lane i + n

// Maximum over the 8 lanes of a block.
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v) {
    v = max(v, dpp_u32<kQuadXor1>(v));
    v = max(v, dpp_u32<kQuadXor2>(v));
    v = max(v, dpp_u32<kHalfRowMirror>(v));
    return v;
}

// Sum of the 128 values of a block in the exact order of ATen's CPU reduction over
// a contiguous row of 128 fp32 values:
//   V[v][l] = r[8v + l];  acc_k[l] = (((0 + V[k][l]) + V[k+4][l]) + V[k+8][l]) + V[k+12][l]
//   A[l] = ((acc_0[l] + acc_1[l]) + acc_2[l]) + acc_3[l];  S = ((0 + A[0]) + A[1]) + ... + A[7]
// Value r[32q + 4j + t] lives in lane j, quarter q, slot t, so acc for offset c = 4j + t
// (= 8k + l) is the lane-local running sum over q: acc[t] = (((0 + r_0) + r_1) + r_2) + r_3
// (accumulated by the caller quarter by quarter).  A[l] gathers lanes l/4, l/4+2, l/4+4,
// l/4+6 and S joins lanes 0 and 1.  The result is valid in lane j == 0.
__device__ __forceinline__ float block_sum_cross(const float (&acc)[4]) {
    float b[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        float s = acc[t] + dpp_f32<kRowShl2>(acc[t]);
        s = s + dpp_f32<kRowShl4>(acc[t]);
        s = s + dpp_f32<kRowShl6>(acc[t]);
        b[t] = s;
    }
    float s = 0.0f + b[0];
    s = s + b[1];
    s = s + b[2];
    s = s + b[3];
    s = s + dpp_f32<kRowShl1>(b[0]);
    s = s + dpp_f32<kRowShl1>(b[1]);
    s = s + dpp_f32<kRowShl1>(b[2]);
    s = s + dpp_f32<kRowShl1>(b[3]);
    return s;
}

// ---------------------------------------------------------------------------
// Philox4x32-10 (Salmon et al., SC'11) streams.  Positions of key `seed` are grouped by
// 128: position P = 128 B + 32 q + 4 j + t (q, t = 0..3, j = 0..7) is the 24-bit field
// i = 4 q + t of the 384-bit little-endian string
//   out(24 B + 3 j) || out(24 B + 3 j + 1) || out(24 B + 3 j + 2),
// out(c) being the four words of Philox(counter = c, key = seed), mapped to [0,1) as
// field * 2^-24.  The lane that owns offsets 32 q + 4 j + t of a 128-value block draws
// its 16 uniforms from three Philox calls, every output bit used once.
// ---------------------------------------------------------------------------

__device__ __forceinline__ void philox4x32_10(uint32_t c0, uint32_t c1, uint32_t k0, uint32_t k1,
                                              uint32_t* out) {
    uint32_t c2 = 0u, c3 = 0u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        // three-input exclusive or in one v_bitop3_b32 (truth table 0x96, symmetric in its inputs)
        const uint32_t n0 = __builtin_amdgcn_bitop3_b32((uint32_t)(p1 >> 32), c1, k0, 0x96);
        const uint32_t n2 = __builtin_amdgcn_bitop3_b32((uint32_t)(p0 >> 32), c3, k1, 0x96);
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

// Philox(counter = ctr, key = seed): four output words.
__device__ __forceinline__ void philox_call(uint64_t seed, uint64_t ctr, uint32_t* w) {
    philox4x32_10((uint32_t)ctr, (uint32_t)(ctr >> 32), (uint32_t)seed, (uint32_t)(seed >> 32), w);
}

// Call r (0..2) of lane j in position group B: words 4r .. 4r+3 of the lane's 384-bit string.
__device__ __forceinline__ void philox_lane_call(uint64_t seed, uint64_t group, int j, int r, uint32_t* w) {
    philox_call(seed, group * 24u + (uint64_t)(3 * j + r), w);
}

// The same call for block grp of a wave tile whose first block is position group g0 (wave-uniform):
// counter 24 (g0 + grp) + 3 j + r = 24 g0 + 3 (8 grp + j) + r, so the 64-bit product is the
// wave's (a scalar one) and each lane adds its small constant.
__device__ __forceinline__ void philox_tile_call(uint64_t seed, uint64_t g0, int grp, int j, int r, uint32_t* w) {
    // The product in scalar registers: read as the first lane's (g0 is the wave tile's, the same in
    // every lane), and held there by an empty asm statement, so that each lane's counter is one
    // 64-bit add rather than two 64-bit vector multiply-adds.
    const uint64_t prod = g0 * 24u;
    uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)prod);
    uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(prod >> 32));
    asm("" : "+s"(lo), "+s"(hi));
    philox_call(seed, ((uint64_t)hi << 32 | lo) + (uint32_t)(24 * grp + 3 * j + r), w);
}

// Fields 4q .. 4q+3 of a lane's string (words 3q .. 3q+2), as exact floats in [0, 2^24):
// the uniforms times 2^24.
// Fields 1 and 2 straddle two words: one byte permute each (v_perm_b32; selector byte k picks
// byte k of the result: 0-3 from the second operand, 4-7 from the first, 0x0C gives 0).
__device__ __forceinline__ void lane_fields4(const uint32_t* w, float (&u)[4]) {
    u[0] = (float)(w[0] & 0xffffffu);
    u[1] = (float)__builtin_amdgcn_perm(w[1], w[0], 0x0C050403u);  // w0 >> 24 | (w1 & 0xffff) << 8
    u[2] = (float)__builtin_amdgcn_perm(w[2], w[1], 0x0C040302u);  // w1 >> 16 | (w2 & 0xff) << 16
    u[3] = (float)(w[2] >> 8);
}

}  // namespace aw4
