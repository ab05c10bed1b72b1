// Fused 4-bit AdamW step for MI355X (gfx950): one multi-tensor launch per optimizer step.
//
// Work decomposition
//   * A 128-value block (one fp32 scale per moment) is owned by 8 lanes of a
//     64-lane wave; a wave owns 8 consecutive blocks (a 1024-value "wave tile").
//   * Lane j (0..7) of a block owns the 16 values at offsets 32q + 4j + t
//     (q, t = 0..3): every parameter/gradient access is a 4-value vector
//     (16 B for fp32) and each quarter q of a block is one contiguous 128 B
//     segment across the 8 lanes.  The same split makes the reference's
//     per-block sum order (ATen's 8-lane x 4-accumulator reduction) mostly
//     lane-local, see eden_sum().
//   * Tiles of all tensors form one index space; each wave walks a contiguous
//     range of it (grid sized to the machine), so one launch covers every
//     parameter of the step, fp32-state tensors included.
//
// Arithmetic contract (bit-for-bit the reference's ATen CPU ops, in order):
//   decode    m = cb[code] * scale                       (_optimized_quantization.py:91-107)
//   moments   m1 = fma(w1, g - m1, m1); m2 = fma(w2, g*g - m2, m2)   (ATen lerp, weight < 0.5)
//   denom     d = sqrt(m2) / sqrt(bc2) + eps             (_optimized.py:219-220)
//   param     p = p * (1 - lr*wd); p = p + (step_coef * m1) / d      (_optimized.py:221-222)
//   encode    s = max(max|m|, 1e-12); x = m / s; round; [dyn4_nz floor]; [EDEN]
//             (_optimized_quantization.py:46-88, _compiled_quantization.py:30-109)
// The file is compiled with -ffp-contract=off: every fused multiply-add is
// written explicitly.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <string>

#include "adamw4bit_hip.h"

namespace {

constexpr int kBlock = AW4_BLOCK;
constexpr int kBlocksPerWave = 8;
constexpr int kWaveTile = kBlock * kBlocksPerWave;  // 1024 values
constexpr int kThreads = 256;
constexpr int kWavesPerGroup = kThreads / 64;
constexpr int kPairs = 17;  // searchsorted-left result 0..16

static_assert(sizeof(aw4_moment) == 72, "aw4_moment layout");
static_assert(sizeof(aw4_tensor) == 208, "aw4_tensor layout");

// Codebooks as fp32 bit patterns (ascending; code = index).  Values of the
// reference's closed forms: NF4 table (quantization.py:401-422), signed and
// unsigned dynamic maps with 3 exponent bits (:201-237), linspace grids (:457-497).
constexpr uint32_t kCodebookBits[AW4_NUM_CODEBOOKS][16] = {
    {0xBF800000u, 0xBF3239B1u, 0xBF066B31u, 0xBECA32A0u, 0xBE91A24Eu, 0xBE3D353Du, 0xBDBA786Cu, 0x00000000u,
     0x3DA2FAFFu, 0x3E24CAE3u, 0x3E7C04DDu, 0x3EAD0339u, 0x3EE1A4B7u, 0x3F1007ABu, 0x3F3913B2u, 0x3F800000u},
    {0xBF633333u, 0xBF29999Au, 0xBEE00000u, 0xBE599999u, 0xBD9EB852u, 0xBD051EB9u, 0xBBB43958u, 0x00000000u,
     0x3BB43958u, 0x3D051EB9u, 0x3D9EB852u, 0x3E599999u, 0x3EE00000u, 0x3F29999Au, 0x3F633333u, 0x3F800000u},
    {0x00000000u, 0x3B54FDF4u, 0x3BFDF3B5u, 0x3CAE147Bu, 0x3D333333u, 0x3D87AE15u, 0x3DB5C28Fu, 0x3E200000u,
     0x3E89999Au, 0x3EC33333u, 0x3EFCCCCDu, 0x3F1B3334u, 0x3F380000u, 0x3F54CCCCu, 0x3F71999Au, 0x3F800000u},
    {0x00000000u, 0x3D888889u, 0x3E088889u, 0x3E4CCCCEu, 0x3E888889u, 0x3EAAAAABu, 0x3ECCCCCEu, 0x3EEEEEF0u,
     0x3F088888u, 0x3F199999u, 0x3F2AAAAAu, 0x3F3BBBBCu, 0x3F4CCCCDu, 0x3F5DDDDEu, 0x3F6EEEEFu, 0x3F800000u},
    {0x3D800000u, 0x3E000000u, 0x3E400000u, 0x3E800000u, 0x3EA00000u, 0x3EC00000u, 0x3EE00000u, 0x3F000000u,
     0x3F100000u, 0x3F200000u, 0x3F300000u, 0x3F400000u, 0x3F500000u, 0x3F600000u, 0x3F700000u, 0x3F800000u},
};

// Lookup-table ids (aw4_encode_tables): round-to-nearest tables then level-count tables.
constexpr int kLutRtn[AW4_NUM_CODEBOOKS] = {0, 1, 2, 3, 4};
constexpr int kLutRtnDyn4Floor = 5;
constexpr int kLutLevels[AW4_NUM_CODEBOOKS] = {6, 7, 8, 9, 10};

// Neighbouring levels of a searchsorted-left index (_compiled_quantization.py:30-38).
struct __align__(16) PairEntry {
    float a;         // cb[lo]
    float b;         // cb[hi]
    float width_rcp; // RN(1 / max(b - a, 1e-12))
    uint32_t lohi;   // lo | hi << 8
};

// Per-block update-SR quantities for each searchsorted index (see update_sr_tables()).
struct __align__(16) UpdEntry {
    float f_hi;   // preconditioner at the upper level
    float den;    // max(f(lo) - f(hi), 1e-30)
    float den_rcp;
    float valid;  // 1 when (b > a) & (f(lo) - f(hi) > 0)
};

struct Tables {
    float codebook[AW4_NUM_CODEBOOKS][16];
    PairEntry pairs[AW4_NUM_CODEBOOKS][kPairs];
    uint2 lut[AW4_NUM_LUTS][AW4_LUT_ENTRIES];  // {threshold bits, base}
};

struct Lds {
    Tables t;
    UpdEntry upd[kWavesPerGroup][kBlocksPerWave][kPairs];
    float pre[kWavesPerGroup][kBlocksPerWave][16];
};

// Launch table staged in device memory: header, tensors[count], tile_start[count + 1].
struct StepHeader {
    int32_t count;
    uint32_t lut_mask;
    int64_t total_tiles;
    int64_t tiles_per_wave;
    int64_t reserved;
};

// ---------------------------------------------------------------------------
// Scalar helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

// ATen clamp_min / clamp propagate NaN.
__device__ __forceinline__ float clamp_min_nan(float x, float lo) { return x < lo ? lo : x; }
__device__ __forceinline__ float clamp01_nan(float x) { return x < 0.0f ? 0.0f : (x > 1.0f ? 1.0f : x); }

// RN(v / s) from y = RN(1 / s): one FMA correction of RN(v * y) gives the
// correctly rounded quotient (Markstein) while the quotient is a normal
// number; subnormal quotients and huge/non-finite divisors take the IEEE
// division.  `slow` must be uniform over the values sharing the divisor.
__device__ __forceinline__ float div_rcp(float v, float s, float y, bool slow) {
    if (slow) return v / s;
    float q = v * y;
    const float r = __builtin_fmaf(-q, s, v);
    q = __builtin_fmaf(r, y, q);
    if (__builtin_expect(fabsf(q) < 0x1p-125f, 0)) q = v / s;
    return q;
}

// bf16 round-to-nearest-even (c10::BFloat16), NaN kept quiet.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    const uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }
// IEEE binary16, round-to-nearest-even (v_cvt_f16_f32), subnormals kept.
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Round an fp32 result to the parameter's storage precision (ATen's in-place
// ops on 16-bit tensors compute in fp32 and round on store).
__device__ __forceinline__ float round_to_storage(float v, int dtype) {
    if (dtype == AW4_BF16) return bf16_to_f32(f32_to_bf16(v));
    if (dtype == AW4_F16) return f16_to_f32(f32_to_f16(v));
    return v;
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
constexpr int kQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kHalfRowMirror = 0x141; // lane i <- lane 7 - i within 8 lanes
template <int n> struct RowShl { static constexpr int value = 0x100 + n; };  // lane i <- lane i + n

// Maximum over the 8 lanes of a block; integer order of |x| bit patterns so a
// NaN propagates like ATen's max reduction.
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v) {
    v = max(v, dpp_u32<kQuadXor1>(v));
    v = max(v, dpp_u32<kQuadXor2>(v));
    v = max(v, dpp_u32<kHalfRowMirror>(v));
    return v;
}

// Sum of the 128 products of a block in the exact order of ATen's CPU
// reduction over a contiguous row of 128 fp32 values:
//   V[v][l] = r[8v + l];  acc_k[l] = (((0 + V[k][l]) + V[k+4][l]) + V[k+8][l]) + V[k+12][l]
//   A[l] = ((acc_0[l] + acc_1[l]) + acc_2[l]) + acc_3[l];  S = ((0 + A[0]) + A[1]) + ... + A[7]
// Value r[32q + 4j + t] lives in lane j, slot 4q + t, so acc for offset
// c = 4j + t (= 8k + l) is lane-local over q, A[l] gathers lanes l/4, l/4+2,
// l/4+4, l/4+6 and S joins lanes 0 and 1.  Result valid in lane j == 0.
__device__ __forceinline__ float eden_sum(const float (&v)[16]) {
    float acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        float a = 0.0f + v[t];
        a = a + v[4 + t];
        a = a + v[8 + t];
        a = a + v[12 + t];
        acc[t] = a;
    }
    float b[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        float s = acc[t] + dpp_f32<RowShl<2>::value>(acc[t]);
        s = s + dpp_f32<RowShl<4>::value>(acc[t]);
        s = s + dpp_f32<RowShl<6>::value>(acc[t]);
        b[t] = s;
    }
    float s = 0.0f + b[0];
    s = s + b[1];
    s = s + b[2];
    s = s + b[3];
    s = s + dpp_f32<RowShl<1>::value>(b[0]);
    s = s + dpp_f32<RowShl<1>::value>(b[1]);
    s = s + dpp_f32<RowShl<1>::value>(b[2]);
    s = s + dpp_f32<RowShl<1>::value>(b[3]);
    return s;
}

// ---------------------------------------------------------------------------
// Philox4x32-10 (Salmon et al., SC'11), counter = draw position / 4.
// ---------------------------------------------------------------------------

__device__ __forceinline__ void philox4x32_10(uint32_t c0, uint32_t c1, uint32_t k0, uint32_t k1, uint32_t (&out)[4]) {
    uint32_t c2 = 0u, c3 = 0u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

// Four uniforms in [0, 1) with 24 random bits each for stream positions pos..pos+3 (pos % 4 == 0).
__device__ __forceinline__ void uniforms4(uint64_t seed, uint64_t pos, float (&u)[4]) {
    const uint64_t ctr = pos >> 2;
    uint32_t r[4];
    philox4x32_10((uint32_t)ctr, (uint32_t)(ctr >> 32), (uint32_t)seed, (uint32_t)(seed >> 32), r);
#pragma unroll
    for (int t = 0; t < 4; ++t) u[t] = (float)(r[t] >> 8) * 0x1p-24f;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Streaming (non-temporal) vector accesses: every byte is touched once per step.
__device__ __forceinline__ f32x4 ld_nt(const float* p) { return __builtin_nontemporal_load((const f32x4*)p); }
__device__ __forceinline__ void st_nt(float* p, f32x4 v) { __builtin_nontemporal_store(v, (f32x4*)p); }
__device__ __forceinline__ u32x2 ld_nt(const uint16_t* p) { return __builtin_nontemporal_load((const u32x2*)p); }
__device__ __forceinline__ void st_nt(uint16_t* p, u32x2 v) { __builtin_nontemporal_store(v, (u32x2*)p); }

// ---------------------------------------------------------------------------
// Memory access helpers (4 consecutive values)
// ---------------------------------------------------------------------------

__device__ __forceinline__ void load4(const void* base, int dtype, int64_t e, bool vec, float (&o)[4]) {
    if (dtype == AW4_F32) {
        const float* p = (const float*)base + e;
        if (vec) {
            const f32x4 v = ld_nt(p);
            o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) o[t] = p[t];
        }
    } else {
        const uint16_t* p = (const uint16_t*)base + e;
        uint16_t h[4];
        if (vec) {
            const u32x2 v = ld_nt(p);
            h[0] = (uint16_t)v.x; h[1] = (uint16_t)(v.x >> 16); h[2] = (uint16_t)v.y; h[3] = (uint16_t)(v.y >> 16);
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) h[t] = p[t];
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) o[t] = dtype == AW4_BF16 ? bf16_to_f32(h[t]) : f16_to_f32(h[t]);
    }
}

__device__ __forceinline__ void store4(void* base, int dtype, int64_t e, bool vec, const float (&v)[4]) {
    if (dtype == AW4_F32) {
        float* p = (float*)base + e;
        if (vec) {
            st_nt(p, f32x4{v[0], v[1], v[2], v[3]});
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) p[t] = v[t];
        }
    } else {
        uint16_t h[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) h[t] = dtype == AW4_BF16 ? f32_to_bf16(v[t]) : f32_to_f16(v[t]);
        uint16_t* p = (uint16_t*)base + e;
        if (vec) {
            st_nt(p, u32x2{(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)});
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) p[t] = h[t];
        }
    }
}

__device__ __forceinline__ float load1(const void* base, int dtype, int64_t e) {
    if (dtype == AW4_F32) return ((const float*)base)[e];
    const uint16_t h = ((const uint16_t*)base)[e];
    return dtype == AW4_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

__device__ __forceinline__ void store1(void* base, int dtype, int64_t e, float v) {
    if (dtype == AW4_F32) ((float*)base)[e] = v;
    else ((uint16_t*)base)[e] = dtype == AW4_BF16 ? f32_to_bf16(v) : f32_to_f16(v);
}

// ---------------------------------------------------------------------------
// Codec
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t lut_index(const uint2* lut, float x) {
    const uint32_t u = f2u(x);
    int k = (int)((u & 0x7fffffffu) >> 20) - (AW4_LUT_EXP0 - 1);
    k = min(max(k, 0), AW4_LUT_HALF - 1);
    const uint2 e = lut[k + (int)(u >> 31) * AW4_LUT_HALF];
    return e.y + (x >= u2f(e.x) ? 1u : 0u);
}

// Decode one block slice: 16 values of lane j from 4 x 16-bit code words.
__device__ __forceinline__ void decode16(const float* cb, const uint32_t (&w)[4], float scale, float (&m)[16]) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int t = 0; t < 4; ++t) m[4 * q + t] = cb[(w[q] >> (4 * t)) & 15u] * scale;
}

struct EncodeCtx {
    const Lds* lds;
    UpdEntry* upd;   // this block's update-SR table (LDS)
    float* pre;      // this block's 16-entry scratch (LDS)
    int j;           // lane within the block
};

// Per-block update-SR tables: for each searchsorted index i, the upper-level
// preconditioner f(hi), the clamped difference f(lo) - f(hi) and its
// reciprocal, and the validity flag of _compiled_quantization.py:199-200, with
// f(l) = 1 / (sqrt(max((s * l) / bias, 0)) + eps)  (:191-193).
__device__ __forceinline__ void update_sr_tables(const EncodeCtx& c, int cbid, float s, float bias, float bias_rcp,
                                                 float eps) {
    const float* cb = c.lds->t.codebook[cbid];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int k = c.j + 8 * h;
        const float vh = clamp_min_nan(div_rcp(s * cb[k], bias, bias_rcp, false), 0.0f);
        c.pre[k] = 1.0f / (sqrtf(vh) + eps);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int h = 0; h < 3; ++h) {
        const int i = c.j + 8 * h;
        if (i < kPairs) {
            const PairEntry pe = c.lds->t.pairs[cbid][i];
            const int lo = (int)(pe.lohi & 0xffu), hi = (int)(pe.lohi >> 8);
            const float flo = c.pre[lo], fhi = c.pre[hi];
            const float den = flo - fhi;
            const float dc = clamp_min_nan(den, 1e-30f);
            UpdEntry u;
            u.f_hi = fhi;
            u.den = dc;
            u.den_rcp = 1.0f / dc;
            u.valid = (pe.b > pe.a && den > 0.0f) ? 1.0f : 0.0f;
            c.upd[i] = u;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Fetch 16 uniforms for this lane's values of block `blk` of a write.
__device__ __forceinline__ void draws16(const aw4_moment& M, int64_t blk, int j, bool active, float (&u)[16]) {
    const int64_t e0 = blk * kBlock + 4 * j;
    if (M.flags & AW4_MOMENT_EXT_DRAWS) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (active) v = ld_nt((const float*)M.draws + e0 + 32 * q);
            u[4 * q] = v.x; u[4 * q + 1] = v.y; u[4 * q + 2] = v.z; u[4 * q + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float r[4];
            uniforms4(M.rng_seed, M.rng_offset + (uint64_t)(e0 + 32 * q), r);
#pragma unroll
            for (int t = 0; t < 4; ++t) u[4 * q + t] = r[t];
        }
    }
}

// Encode this lane's 16 values of block `blk` into codes + block scale and
// store them (_optimized_quantization.py:46-88 + pack_4bit_codes).
__device__ __forceinline__ void encode_store(const aw4_moment& M, const EncodeCtx& c, int64_t blk, bool active,
                                             const float (&m)[16]) {
    const int cbid = M.codebook;
    // Block absmax, floored at 1e-12 (NaN-propagating integer max of |m| bits).
    uint32_t amax = 0u;
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = max(amax, f2u(m[i]) & 0x7fffffffu);
    amax = block_max_u32(amax);
    const float s = u2f(max(amax, 0x2B8CBCCCu));  // 0x2B8CBCCC = fp32(1e-12)
    const bool slow = !(s < 0x1p125f);
    const float y = 1.0f / s;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = div_rcp(m[i], s, y, slow);

    uint32_t code[16];
    const int rounding = M.rounding;
    if (rounding == AW4_ROUND_RTN) {
        const uint2* lut = c.lds->t.lut[(M.flags & AW4_MOMENT_ZERO_FLOOR) && cbid == AW4_CB_DYN4
                                            ? kLutRtnDyn4Floor : kLutRtn[cbid]];
#pragma unroll
        for (int i = 0; i < 16; ++i) code[i] = lut_index(lut, x[i]);
        if ((M.flags & AW4_MOMENT_ZERO_FLOOR) && cbid != AW4_CB_DYN4) {
#pragma unroll
            for (int i = 0; i < 16; ++i) code[i] = max(code[i], 1u);
        }
    } else {
        float u[16];
        draws16(M, blk, c.j, active, u);
        const uint2* lut = c.lds->t.lut[kLutLevels[cbid]];
        const PairEntry* pairs = c.lds->t.pairs[cbid];
        const bool guards = (M.flags & AW4_MOMENT_GUARDS) != 0;
        if (rounding == AW4_ROUND_STATE_SR) {
            // P(hi) = (x - a) / max(b - a, 1e-12), 0 where b == a; clamp; guards x<=a -> 0, x>=b -> 1
            // (_compiled_quantization.py:60-71).
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const PairEntry pe = pairs[lut_index(lut, x[i])];
                const float width = pe.b - pe.a;
                float p = div_rcp(x[i] - pe.a, width < 1e-12f ? 1e-12f : width, pe.width_rcp, false);
                p = width > 0.0f ? p : 0.0f;
                p = clamp01_nan(p);
                if (guards) {
                    p = x[i] >= pe.b ? 1.0f : p;
                    p = x[i] <= pe.a ? 0.0f : p;
                }
                code[i] = u[i] < p ? (pe.lohi >> 8) : (pe.lohi & 0xffu);
            }
        } else {
            // P(lo) = (f(x) - f(b)) / max(f(a) - f(b), 1e-30), 1 unless b > a and f(a) > f(b);
            // clamp; guards x<=a -> 1, x>=b -> 0 (_compiled_quantization.py:74-109).
            update_sr_tables(c, cbid, s, M.sr_bias, M.sr_bias_rcp, M.sr_eps);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t idx = lut_index(lut, x[i]);
                const PairEntry pe = pairs[idx];
                const UpdEntry ue = c.upd[idx];
                const float vh = clamp_min_nan(div_rcp(s * x[i], M.sr_bias, M.sr_bias_rcp, false), 0.0f);
                const float fx = 1.0f / (sqrtf(vh) + M.sr_eps);
                float p = div_rcp(fx - ue.f_hi, ue.den, ue.den_rcp, false);
                p = ue.valid != 0.0f ? p : 1.0f;
                p = clamp01_nan(p);
                if (guards) {
                    p = x[i] >= pe.b ? 0.0f : p;
                    p = x[i] <= pe.a ? 1.0f : p;
                }
                code[i] = u[i] < p ? (pe.lohi & 0xffu) : (pe.lohi >> 8);
            }
        }
        if (M.flags & AW4_MOMENT_ZERO_FLOOR) {
#pragma unroll
            for (int i = 0; i < 16; ++i) code[i] = max(code[i], 1u);
        }
    }

    float scale = s;
    if (M.flags & AW4_MOMENT_EDEN) {
        // s' = s * (sum x*x / max(sum x*cb[code], 1e-12))  (_optimized_quantization.py:81-85)
        const float* cb = c.lds->t.codebook[cbid];
        float xx[16], xl[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            xx[i] = x[i] * x[i];
            xl[i] = x[i] * cb[code[i]];
        }
        const float num = eden_sum(xx);
        const float den = eden_sum(xl);
        scale = s * (num / clamp_min_nan(den, 1e-12f));
    }

    if (active) {
        uint8_t* codes = (uint8_t*)M.codes + blk * (kBlock / 2) + 2 * c.j;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t w = code[4 * q] | (code[4 * q + 1] << 4) | (code[4 * q + 2] << 8) | (code[4 * q + 3] << 12);
            *(uint16_t*)(codes + 16 * q) = (uint16_t)w;
        }
        if (c.j == 0) ((float*)M.scales)[blk] = scale;
    }
}

// Load this lane's 16 values of moment M for block `blk` (decoded if quantized).
__device__ __forceinline__ void load_moment(const aw4_moment& M, const Lds& lds, int64_t blk, int j, bool active,
                                            float (&m)[16]) {
    const int64_t e0 = blk * kBlock + 4 * j;
    if (M.rounding == AW4_ROUND_FP32) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (active) v = ld_nt((const float*)M.values + e0 + 32 * q);
            m[4 * q] = v.x; m[4 * q + 1] = v.y; m[4 * q + 2] = v.z; m[4 * q + 3] = v.w;
        }
    } else {
        uint32_t w[4] = {0u, 0u, 0u, 0u};
        float scale = 0.0f;
        if (active) {
            const uint8_t* codes = (const uint8_t*)M.codes + blk * (kBlock / 2) + 2 * j;
#pragma unroll
            for (int q = 0; q < 4; ++q) w[q] = *(const uint16_t*)(codes + 16 * q);
            scale = ((const float*)M.scales)[blk];
        }
        decode16(lds.t.codebook[M.codebook], w, scale, m);
    }
}

__device__ __forceinline__ void store_moment_fp32(const aw4_moment& M, int64_t blk, int j, bool active,
                                                  const float (&m)[16]) {
    if (!active) return;
    const int64_t e0 = blk * kBlock + 4 * j;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        st_nt((float*)M.values + e0 + 32 * q, f32x4{m[4 * q], m[4 * q + 1], m[4 * q + 2], m[4 * q + 3]});
}

// The AdamW arithmetic of one value (_optimized.py:215-222), in ATen's order.
__device__ __forceinline__ void adamw_value(const aw4_tensor& T, float g, float& m1, float& m2, float& p) {
    const float gg = g * g;
    m1 = (T.flags & AW4_TENSOR_LERP1_LARGE) ? __builtin_fmaf(T.w1, g - m1, g) : __builtin_fmaf(T.w1, g - m1, m1);
    m2 = (T.flags & AW4_TENSOR_LERP2_LARGE) ? __builtin_fmaf(T.w2, gg - m2, gg) : __builtin_fmaf(T.w2, gg - m2, m2);
    const float d = div_rcp(sqrtf(m2), T.bc2_sqrt, T.bc2_sqrt_rcp, false) + T.eps;
    const float p1 = round_to_storage(p * T.decay, T.param_dtype);
    p = p1 + (T.step_coef * m1) / d;
}

// One wave tile of a tensor whose numel is a multiple of 128: blocks blk0 .. blk0+7.
__device__ void step_tile_blocks(const aw4_tensor& T, int64_t blk0, const Lds& lds, UpdEntry (*upd)[kPairs],
                                 float (*pre)[16], int lane) {
    const int j = lane & 7;
    const int grp = lane >> 3;
    const int64_t blk = blk0 + grp;
    const bool active = blk < (T.numel >> 7);
    const int64_t e0 = blk * kBlock + 4 * j;
    const bool vec = (T.flags & AW4_TENSOR_VEC_ALIGNED) != 0;

    float g[16], p[16], m1[16], m2[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float gv[4] = {0.f, 0.f, 0.f, 0.f}, pv[4] = {0.f, 0.f, 0.f, 0.f};
        if (active) {
            load4((const void*)T.grad, T.grad_dtype, e0 + 32 * q, vec, gv);
            load4((const void*)T.param, T.param_dtype, e0 + 32 * q, vec, pv);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) { g[4 * q + t] = gv[t]; p[4 * q + t] = pv[t]; }
    }
    load_moment(T.m1, lds, blk, j, active, m1);
    load_moment(T.m2, lds, blk, j, active, m2);

#pragma unroll
    for (int i = 0; i < 16; ++i) adamw_value(T, g[i], m1[i], m2[i], p[i]);

    if (active) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float pv[4] = {p[4 * q], p[4 * q + 1], p[4 * q + 2], p[4 * q + 3]};
            store4((void*)T.param, T.param_dtype, e0 + 32 * q, vec, pv);
        }
    }

    const EncodeCtx c{&lds, upd[grp], pre[grp], j};
    if (T.m1.rounding == AW4_ROUND_FP32) store_moment_fp32(T.m1, blk, j, active, m1);
    else encode_store(T.m1, c, blk, active, m1);
    if (T.m2.rounding == AW4_ROUND_FP32) store_moment_fp32(T.m2, blk, j, active, m2);
    else encode_store(T.m2, c, blk, active, m2);
}

// One wave tile of a tensor with fp32 state and arbitrary numel (values e_tile .. e_tile+1023).
__device__ void step_tile_values(const aw4_tensor& T, int64_t e_tile, int lane) {
    const int j = lane & 7;
    const int grp = lane >> 3;
    const bool vec = (T.flags & AW4_TENSOR_VEC_ALIGNED) != 0;
    float* v1 = (float*)T.m1.values;
    float* v2 = (float*)T.m2.values;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t e = e_tile + grp * kBlock + 32 * q + 4 * j;
        if (e >= T.numel) continue;
        if (e + 4 <= T.numel) {
            float g[4], p[4], a[4], b[4];
            load4((const void*)T.grad, T.grad_dtype, e, vec, g);
            load4((const void*)T.param, T.param_dtype, e, vec, p);
            load4(v1, AW4_F32, e, true, a);
            load4(v2, AW4_F32, e, true, b);
#pragma unroll
            for (int t = 0; t < 4; ++t) adamw_value(T, g[t], a[t], b[t], p[t]);
            store4((void*)T.param, T.param_dtype, e, vec, p);
            store4(v1, AW4_F32, e, true, a);
            store4(v2, AW4_F32, e, true, b);
        } else {
            for (int64_t k = e; k < T.numel; ++k) {  // the last 1..3 values of the tensor
                float g = load1((const void*)T.grad, T.grad_dtype, k);
                float p = load1((const void*)T.param, T.param_dtype, k);
                float a = v1[k], b = v2[k];
                adamw_value(T, g, a, b, p);
                store1((void*)T.param, T.param_dtype, k, p);
                v1[k] = a;
                v2[k] = b;
            }
        }
    }
}

__device__ void load_tables(Lds& lds, const Tables* g, uint32_t lut_mask) {
    const int tid = threadIdx.x;
    // codebooks + pair tables (always), then the lookup tables named in the mask
    {
        const uint32_t* src = (const uint32_t*)g;
        uint32_t* dst = (uint32_t*)&lds.t;
        constexpr int kHead = (int)(offsetof(Tables, lut) / 4);
        for (int i = tid; i < kHead; i += kThreads) dst[i] = src[i];
    }
    for (int l = 0; l < AW4_NUM_LUTS; ++l) {
        if (!(lut_mask & (1u << l))) continue;
        const uint2* src = g->lut[l];
        uint2* dst = lds.t.lut[l];
        for (int i = tid; i < AW4_LUT_ENTRIES; i += kThreads) dst[i] = src[i];
    }
    __syncthreads();
}

__global__ void __launch_bounds__(kThreads) fused_step_kernel(const StepHeader* __restrict__ hdr,
                                                              const Tables* __restrict__ tables) {
    __shared__ Lds lds;
    load_tables(lds, tables, hdr->lut_mask);

    const aw4_tensor* tensors = (const aw4_tensor*)(hdr + 1);
    const int64_t* tile_start = (const int64_t*)(tensors + hdr->count);
    const int lane = threadIdx.x & 63;
    const int wslot = threadIdx.x >> 6;
    const int64_t wave = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * kWavesPerGroup + wslot));
    const int64_t total = hdr->total_tiles;
    int64_t tile = wave * hdr->tiles_per_wave;
    const int64_t end = min(tile + hdr->tiles_per_wave, total);
    if (tile >= end) return;

    // tensor containing `tile`: last ti with tile_start[ti] <= tile
    int lo = 0, hi = hdr->count - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tile_start[mid] <= tile) lo = mid; else hi = mid - 1;
    }
    int ti = lo;
    for (; tile < end; ++tile) {
        while (tile >= tile_start[ti + 1]) ++ti;
        const aw4_tensor& T = tensors[ti];
        const int64_t local = tile - tile_start[ti];
        if ((T.numel & (kBlock - 1)) == 0)
            step_tile_blocks(T, local * kBlocksPerWave, lds, lds.upd[wslot], lds.pre[wslot], lane);
        else
            step_tile_values(T, local * kWaveTile, lane);
    }
}

// Stand-alone codec kernels (one wave tile per wave, grid-stride).
__global__ void __launch_bounds__(kThreads) quantize_kernel(const float* __restrict__ values, int64_t numel,
                                                            aw4_moment M, const Tables* __restrict__ tables,
                                                            uint32_t lut_mask) {
    __shared__ Lds lds;
    load_tables(lds, tables, lut_mask);
    const int lane = threadIdx.x & 63;
    const int wslot = threadIdx.x >> 6;
    const int j = lane & 7, grp = lane >> 3;
    const int64_t nblocks = numel / kBlock;
    const int64_t tiles = (nblocks + kBlocksPerWave - 1) / kBlocksPerWave;
    const int64_t nwaves = (int64_t)gridDim.x * kWavesPerGroup;
    for (int64_t tile = (int64_t)blockIdx.x * kWavesPerGroup + wslot; tile < tiles; tile += nwaves) {
        const int64_t blk = tile * kBlocksPerWave + grp;
        const bool active = blk < nblocks;
        float m[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (active) v = *(const float4*)(values + blk * kBlock + 32 * q + 4 * j);
            m[4 * q] = v.x; m[4 * q + 1] = v.y; m[4 * q + 2] = v.z; m[4 * q + 3] = v.w;
        }
        const EncodeCtx c{&lds, lds.upd[wslot][grp], lds.pre[wslot][grp], j};
        encode_store(M, c, blk, active, m);
    }
}

__global__ void __launch_bounds__(kThreads) dequantize_kernel(aw4_moment M, int64_t numel, float* __restrict__ out,
                                                              const Tables* __restrict__ tables) {
    __shared__ Lds lds;
    load_tables(lds, tables, 0u);
    const int lane = threadIdx.x & 63;
    const int wslot = threadIdx.x >> 6;
    const int j = lane & 7, grp = lane >> 3;
    const int64_t nblocks = numel / kBlock;
    const int64_t tiles = (nblocks + kBlocksPerWave - 1) / kBlocksPerWave;
    const int64_t nwaves = (int64_t)gridDim.x * kWavesPerGroup;
    for (int64_t tile = (int64_t)blockIdx.x * kWavesPerGroup + wslot; tile < tiles; tile += nwaves) {
        const int64_t blk = tile * kBlocksPerWave + grp;
        const bool active = blk < nblocks;
        float m[16];
        load_moment(M, lds, blk, j, active, m);
        if (active) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *(float4*)(out + blk * kBlock + 32 * q + 4 * j) =
                    make_float4(m[4 * q], m[4 * q + 1], m[4 * q + 2], m[4 * q + 3]);
        }
    }
}

__global__ void __launch_bounds__(kThreads) uniforms_kernel(uint64_t seed, uint64_t offset, int64_t n,
                                                            float* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * kThreads * 4;
    for (int64_t e = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 4; e < n; e += stride) {
        float u[4];
        uniforms4(seed, offset + (uint64_t)e, u);
#pragma unroll
        for (int t = 0; t < 4; ++t)
            if (e + t < n) out[e + t] = u[t];
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

thread_local std::string g_error;

int set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

#define AW4_HIP_CHECK(expr)                                                                  \
    do {                                                                                     \
        hipError_t err_ = (expr);                                                            \
        if (err_ != hipSuccess) return set_error(AW4_EHIP, "%s: %s", #expr, hipGetErrorString(err_)); \
    } while (0)

float host_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
uint32_t host_u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

int count_less(const float* cb, float x) {
    int c = 0;
    for (int k = 0; k < 16; ++k) c += cb[k] < x ? 1 : 0;
    return c;
}

// Round-to-nearest code of the reference (ties to the upper level), in fp32.
int rtn_code(const float* cb, float x, bool floor_zero) {
    const int idx = count_less(cb, x);
    const int lo = idx > 0 ? idx - 1 : 0;
    const int hi = idx < 15 ? idx : 15;
    const float da = fabsf(x - cb[lo]);
    const float db = fabsf(cb[hi] - x);
    int code = da < db ? lo : hi;
    if (floor_zero && code == 0) code = 1;
    return code;
}

struct HostTables {
    Tables t;
    bool ok = false;
    std::string error;
};

// Build one lookup table: bucket -> (threshold, base) such that f(x) = base + (x >= threshold)
// for every fp32 x of the bucket, where f is monotone non-decreasing in x.
template <class F>
bool build_lut(uint2* out, F f, std::string& err) {
    for (int sign = 0; sign < 2; ++sign) {
        for (int k = 0; k < AW4_LUT_HALF; ++k) {
            uint32_t alo, ahi;
            if (k == 0) {
                alo = 0u;
                ahi = ((uint32_t)AW4_LUT_EXP0 << 20) - 1u;
            } else if (k < AW4_LUT_HALF - 1) {
                alo = (uint32_t)(AW4_LUT_EXP0 - 1 + k) << 20;
                ahi = alo + (1u << 20) - 1u;
            } else {
                alo = (uint32_t)(AW4_LUT_EXP0 - 1 + k) << 20;
                ahi = 0x7f800000u;
            }
            auto val = [&](uint32_t a) { return sign ? -host_f(a) : host_f(a); };
            // x increases with a for sign 0 and decreases for sign 1
            const uint32_t amin = sign ? ahi : alo, amax = sign ? alo : ahi;
            const int base = f(val(amin));
            const int top = f(val(amax));
            uint2 e;
            e.y = (uint32_t)base;
            if (top == base) {
                e.x = 0x7f800000u;  // +inf: never increments
            } else if (top == base + 1) {
                // smallest x (in value order) with f(x) == base + 1
                uint32_t good = amax, bad = amin;  // f(val(good)) == base+1, f(val(bad)) == base
                while (good != bad && (sign ? bad - good : good - bad) > 1u) {
                    const uint32_t mid = sign ? good + (bad - good) / 2u : bad + (good - bad) / 2u;
                    if (f(val(mid)) == base + 1) good = mid; else bad = mid;
                }
                e.x = host_u(val(good));
            } else {
                char buf[160];
                snprintf(buf, sizeof(buf), "lookup bucket %d (sign %d) spans %d code changes", k, sign, top - base);
                err = buf;
                return false;
            }
            out[k + sign * AW4_LUT_HALF] = e;
        }
    }
    return true;
}

const HostTables& host_tables() {
    static HostTables h;
    static std::once_flag once;
    std::call_once(once, [] {
        Tables& t = h.t;
        memset(&t, 0, sizeof(t));
        for (int c = 0; c < AW4_NUM_CODEBOOKS; ++c) {
            for (int k = 0; k < 16; ++k) t.codebook[c][k] = host_f(kCodebookBits[c][k]);
            for (int i = 0; i < kPairs; ++i) {
                const int lo = i > 0 ? i - 1 : 0, hi = i < 15 ? i : 15;
                PairEntry& p = t.pairs[c][i];
                p.a = t.codebook[c][lo];
                p.b = t.codebook[c][hi];
                const float w = p.b - p.a;
                p.width_rcp = 1.0f / (w < 1e-12f ? 1e-12f : w);
                p.lohi = (uint32_t)lo | ((uint32_t)hi << 8);
            }
        }
        bool ok = true;
        for (int c = 0; c < AW4_NUM_CODEBOOKS && ok; ++c) {
            const float* cb = t.codebook[c];
            ok = build_lut(t.lut[kLutRtn[c]], [cb](float x) { return rtn_code(cb, x, false); }, h.error) &&
                 build_lut(t.lut[kLutLevels[c]], [cb](float x) { return count_less(cb, x); }, h.error);
        }
        if (ok) {
            const float* cb = t.codebook[AW4_CB_DYN4];
            ok = build_lut(t.lut[kLutRtnDyn4Floor], [cb](float x) { return rtn_code(cb, x, true); }, h.error);
        }
        h.ok = ok;
    });
    return h;
}

struct StagingSlot {
    void* host = nullptr;
    void* dev = nullptr;
    size_t cap = 0;
    hipEvent_t done = nullptr;
    bool pending = false;
};

constexpr int kSlots = 4;

struct DeviceState {
    Tables* tables = nullptr;
    int num_cus = 0;
    StagingSlot slots[kSlots];
    int next = 0;
};

std::mutex g_mutex;
std::map<int, DeviceState> g_devices;

int device_state(DeviceState** out) {
    const HostTables& ht = host_tables();
    if (!ht.ok) return set_error(AW4_EINVAL, "encode tables: %s", ht.error.c_str());
    int dev = 0;
    AW4_HIP_CHECK(hipGetDevice(&dev));
    DeviceState& ds = g_devices[dev];
    if (!ds.tables) {
        hipDeviceProp_t prop;
        AW4_HIP_CHECK(hipGetDeviceProperties(&prop, dev));
        ds.num_cus = prop.multiProcessorCount;
        Tables* d = nullptr;
        AW4_HIP_CHECK(hipMalloc((void**)&d, sizeof(Tables)));
        hipError_t e = hipMemcpy(d, &ht.t, sizeof(Tables), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            (void)hipFree(d);
            return set_error(AW4_EHIP, "hipMemcpy(tables): %s", hipGetErrorString(e));
        }
        ds.tables = d;
    }
    *out = &ds;
    return AW4_OK;
}

uint32_t lut_mask_for(const aw4_moment& m) {
    if (m.rounding == AW4_ROUND_FP32) return 0u;
    if (m.rounding == AW4_ROUND_RTN) {
        if ((m.flags & AW4_MOMENT_ZERO_FLOOR) && m.codebook == AW4_CB_DYN4) return 1u << kLutRtnDyn4Floor;
        return 1u << kLutRtn[m.codebook];
    }
    return 1u << kLutLevels[m.codebook];
}

bool aligned(uint64_t addr, uint64_t a) { return (addr % a) == 0; }

int check_moment(const aw4_moment& m, int64_t numel, int index, const char* name) {
    if (m.rounding == AW4_ROUND_FP32) {
        if (!m.values) return set_error(AW4_EINVAL, "tensor %d: %s fp32 state without values", index, name);
        if (!aligned(m.values, 16)) return set_error(AW4_EALIGN, "tensor %d: %s values not 16-byte aligned", index, name);
        return AW4_OK;
    }
    if (m.rounding < AW4_ROUND_RTN || m.rounding > AW4_ROUND_UPDATE_SR)
        return set_error(AW4_EINVAL, "tensor %d: %s has rounding %d", index, name, m.rounding);
    if (m.codebook < 0 || m.codebook >= AW4_NUM_CODEBOOKS)
        return set_error(AW4_EINVAL, "tensor %d: %s has codebook %d", index, name, m.codebook);
    if (numel % kBlock != 0)
        return set_error(AW4_EINVAL, "tensor %d: %s quantized but numel %lld is not a multiple of %d", index, name,
                         (long long)numel, kBlock);
    if (!m.codes || !m.scales) return set_error(AW4_EINVAL, "tensor %d: %s quantized without codes/scales", index, name);
    if (!aligned(m.codes, 2) || !aligned(m.scales, 4))
        return set_error(AW4_EALIGN, "tensor %d: %s codes/scales misaligned", index, name);
    if (m.rounding != AW4_ROUND_RTN) {
        if (m.flags & AW4_MOMENT_EXT_DRAWS) {
            if (!m.draws || !aligned(m.draws, 16))
                return set_error(AW4_EINVAL, "tensor %d: %s external draws missing or misaligned", index, name);
        } else if (m.rng_offset % 4 != 0) {
            return set_error(AW4_EINVAL, "tensor %d: %s rng_offset not a multiple of 4", index, name);
        }
    }
    if (m.rounding == AW4_ROUND_UPDATE_SR && !(m.sr_bias > 0.0f))
        return set_error(AW4_EINVAL, "tensor %d: %s update-SR bias must be positive", index, name);
    return AW4_OK;
}

int check_tensor(const aw4_tensor& t, int index) {
    if (!t.param || !t.grad) return set_error(AW4_EINVAL, "tensor %d: null param or grad", index);
    if (t.numel <= 0) return set_error(AW4_EINVAL, "tensor %d: numel %lld", index, (long long)t.numel);
    for (int dt : {t.param_dtype, t.grad_dtype})
        if (dt != AW4_F32 && dt != AW4_BF16 && dt != AW4_F16)
            return set_error(AW4_EINVAL, "tensor %d: dtype %d", index, dt);
    if (t.flags & AW4_TENSOR_VEC_ALIGNED) {
        const uint64_t pa = t.param_dtype == AW4_F32 ? 16 : 8, ga = t.grad_dtype == AW4_F32 ? 16 : 8;
        if (!aligned(t.param, pa) || !aligned(t.grad, ga))
            return set_error(AW4_EALIGN, "tensor %d: VEC_ALIGNED but param/grad misaligned", index);
    }
    int rc = check_moment(t.m1, t.numel, index, "m1");
    if (rc) return rc;
    return check_moment(t.m2, t.numel, index, "m2");
}

int stream_launch_grid(const DeviceState& ds, int64_t waves_needed, int64_t* waves) {
    // Enough waves to fill the machine several times over, no more than the work.
    const int64_t target = (int64_t)ds.num_cus * 32;
    *waves = waves_needed < target ? waves_needed : target;
    return AW4_OK;
}

}  // namespace

extern "C" {

int aw4_abi_version(void) { return AW4_ABI_VERSION; }

const char* aw4_last_error(void) { return g_error.c_str(); }

int64_t aw4_encode_tables(void* out, int64_t bytes) {
    const HostTables& ht = host_tables();
    if (!ht.ok) return set_error(AW4_EINVAL, "encode tables: %s", ht.error.c_str());
    const int64_t size = (int64_t)sizeof(ht.t.lut);
    if (!out) return size;
    if (bytes < size) return set_error(AW4_EINVAL, "aw4_encode_tables: need %lld bytes", (long long)size);
    memcpy(out, ht.t.lut, (size_t)size);
    return size;
}

int aw4_fused_step(const aw4_tensor* tensors, int32_t count, void* stream) {
    g_error.clear();
    if (count < 0 || (count > 0 && !tensors)) return set_error(AW4_EINVAL, "aw4_fused_step: bad tensor list");
    if (count == 0) return AW4_OK;
    uint32_t mask = 0u;
    int64_t total = 0;
    for (int i = 0; i < count; ++i) {
        const int rc = check_tensor(tensors[i], i);
        if (rc) return rc;
        mask |= lut_mask_for(tensors[i].m1) | lut_mask_for(tensors[i].m2);
        total += (tensors[i].numel + kWaveTile - 1) / kWaveTile;
    }
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceState* ds = nullptr;
    int rc = device_state(&ds);
    if (rc) return rc;

    int64_t waves = 0;
    stream_launch_grid(*ds, total, &waves);
    const int64_t per_wave = (total + waves - 1) / waves;
    waves = (total + per_wave - 1) / per_wave;
    const int64_t groups = (waves + kWavesPerGroup - 1) / kWavesPerGroup;

    const size_t bytes = sizeof(StepHeader) + sizeof(aw4_tensor) * (size_t)count + sizeof(int64_t) * (size_t)(count + 1);
    StagingSlot& slot = ds->slots[ds->next];
    ds->next = (ds->next + 1) % kSlots;
    if (slot.pending) {
        AW4_HIP_CHECK(hipEventSynchronize(slot.done));
        slot.pending = false;
    }
    if (slot.cap < bytes) {
        if (slot.host) AW4_HIP_CHECK(hipHostFree(slot.host));
        if (slot.dev) AW4_HIP_CHECK(hipFree(slot.dev));
        slot.host = slot.dev = nullptr;
        slot.cap = 0;
        size_t cap = 4096;
        while (cap < bytes) cap *= 2;
        AW4_HIP_CHECK(hipHostMalloc(&slot.host, cap, hipHostMallocDefault));
        AW4_HIP_CHECK(hipMalloc(&slot.dev, cap));
        slot.cap = cap;
    }
    if (!slot.done) AW4_HIP_CHECK(hipEventCreateWithFlags(&slot.done, hipEventDisableTiming));

    StepHeader* h = (StepHeader*)slot.host;
    h->count = count;
    h->lut_mask = mask;
    h->total_tiles = total;
    h->tiles_per_wave = per_wave;
    h->reserved = 0;
    memcpy(h + 1, tensors, sizeof(aw4_tensor) * (size_t)count);
    int64_t* starts = (int64_t*)((aw4_tensor*)(h + 1) + count);
    int64_t acc = 0;
    for (int i = 0; i < count; ++i) {
        starts[i] = acc;
        acc += (tensors[i].numel + kWaveTile - 1) / kWaveTile;
    }
    starts[count] = acc;

    hipStream_t s = (hipStream_t)stream;
    AW4_HIP_CHECK(hipMemcpyAsync(slot.dev, slot.host, bytes, hipMemcpyHostToDevice, s));
    hipLaunchKernelGGL(fused_step_kernel, dim3((unsigned)groups), dim3(kThreads), 0, s, (const StepHeader*)slot.dev,
                       (const Tables*)ds->tables);
    AW4_HIP_CHECK(hipGetLastError());
    AW4_HIP_CHECK(hipEventRecord(slot.done, s));
    slot.pending = true;
    return AW4_OK;
}

int aw4_quantize(const float* values, int64_t numel, const aw4_moment* m, void* stream) {
    g_error.clear();
    if (!values || !m || numel <= 0 || numel % kBlock != 0)
        return set_error(AW4_EINVAL, "aw4_quantize: bad arguments (numel %lld)", (long long)numel);
    if (((uint64_t)values) % 16 != 0) return set_error(AW4_EALIGN, "aw4_quantize: values not 16-byte aligned");
    if (m->rounding == AW4_ROUND_FP32) return set_error(AW4_EINVAL, "aw4_quantize: fp32 moment");
    int rc = check_moment(*m, numel, 0, "moment");
    if (rc) return rc;
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceState* ds = nullptr;
    rc = device_state(&ds);
    if (rc) return rc;
    const int64_t tiles = (numel / kBlock + kBlocksPerWave - 1) / kBlocksPerWave;
    int64_t groups = (tiles + kWavesPerGroup - 1) / kWavesPerGroup;
    if (groups > (int64_t)ds->num_cus * 8) groups = (int64_t)ds->num_cus * 8;
    hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)groups), dim3(kThreads), 0, (hipStream_t)stream, values, numel,
                       *m, (const Tables*)ds->tables, lut_mask_for(*m));
    AW4_HIP_CHECK(hipGetLastError());
    return AW4_OK;
}

int aw4_dequantize(const aw4_moment* m, int64_t numel, float* out, void* stream) {
    g_error.clear();
    if (!m || !out || numel <= 0 || numel % kBlock != 0)
        return set_error(AW4_EINVAL, "aw4_dequantize: bad arguments (numel %lld)", (long long)numel);
    if (((uint64_t)out) % 16 != 0) return set_error(AW4_EALIGN, "aw4_dequantize: out not 16-byte aligned");
    if (m->rounding == AW4_ROUND_FP32) return set_error(AW4_EINVAL, "aw4_dequantize: fp32 moment");
    if (m->codebook < 0 || m->codebook >= AW4_NUM_CODEBOOKS || !m->codes || !m->scales)
        return set_error(AW4_EINVAL, "aw4_dequantize: bad moment");
    if (!aligned(m->codes, 2) || !aligned(m->scales, 4)) return set_error(AW4_EALIGN, "aw4_dequantize: misaligned");
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceState* ds = nullptr;
    int rc = device_state(&ds);
    if (rc) return rc;
    const int64_t tiles = (numel / kBlock + kBlocksPerWave - 1) / kBlocksPerWave;
    int64_t groups = (tiles + kWavesPerGroup - 1) / kWavesPerGroup;
    if (groups > (int64_t)ds->num_cus * 8) groups = (int64_t)ds->num_cus * 8;
    hipLaunchKernelGGL(dequantize_kernel, dim3((unsigned)groups), dim3(kThreads), 0, (hipStream_t)stream, *m, numel,
                       out, (const Tables*)ds->tables);
    AW4_HIP_CHECK(hipGetLastError());
    return AW4_OK;
}

int aw4_uniforms(uint64_t seed, uint64_t offset, int64_t n, float* out, void* stream) {
    g_error.clear();
    if (!out || n < 0 || offset % 4 != 0) return set_error(AW4_EINVAL, "aw4_uniforms: bad arguments");
    if (n == 0) return AW4_OK;
    int dev = 0;
    AW4_HIP_CHECK(hipGetDevice(&dev));
    int64_t groups = (n / 4 + kThreads - 1) / kThreads;
    if (groups > 4096) groups = 4096;
    hipLaunchKernelGGL(uniforms_kernel, dim3((unsigned)groups), dim3(kThreads), 0, (hipStream_t)stream, seed, offset,
                       n, out);
    AW4_HIP_CHECK(hipGetLastError());
    return AW4_OK;
}

}  // extern "C"
