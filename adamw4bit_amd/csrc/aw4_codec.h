// 4-bit block codec of the fused step: codebook tables, decode, and encode with
// round-to-nearest, value-space or preconditioner-space stochastic rounding.
//
// Block layout: a 128-value block is owned by 8 lanes; lane j holds the 16 values at
// offsets 32q + 4j + t (q, t = 0..3).  Its codes are 4 little-endian 16-bit words
// (word q at byte offset 16q + 2j of the block's 64 code bytes; nibble t = value t).
#pragma once

#include "aw4_math.h"
#include "adamw4bit_hip.h"

namespace aw4 {

constexpr int kBlock = AW4_BLOCK;
constexpr int kPairs = 17;          // searchsorted-left results 0..16
constexpr int kBlocksPerWave = 8;   // a wave tile: 8 blocks, 8 lanes per block

// Rounding kinds (AW4_ROUND_*) and "any": the kind is read from the descriptor at run time.
enum : int { K_FP32 = AW4_ROUND_FP32, K_RTN = AW4_ROUND_RTN, K_SSR = AW4_ROUND_STATE_SR,
             K_USR = AW4_ROUND_UPDATE_SR, K_LA = AW4_ROUND_LOOKAHEAD_SR, K_ANY = 7 };

// Whether a moment keeps codes and scales in memory (a pending lookahead m2 keeps fp32
// values but is still processed block by block).
__host__ __device__ inline bool has_codes(int rounding, int flags) {
    return rounding != K_FP32 && !(rounding == K_LA && (flags & AW4_MOMENT_PENDING));
}

// A moment's compile-time specification: its rounding kind and the AW4_MOMENT_* flags a
// specialised kernel is built for (zero floor, EDEN, guards; external draws stay a run-time
// choice).  kFlagsAtRunTime, a bit above every AW4_MOMENT_* flag, makes the encoder read the
// flags from the descriptor instead.
constexpr int kFlagsAtRunTime = 0x1000;
static_assert(kFlagsAtRunTime > (AW4_MOMENT_ZERO_FLOOR | AW4_MOMENT_EDEN | AW4_MOMENT_GUARDS | AW4_MOMENT_EXT_DRAWS |
                                 AW4_MOMENT_SAMPLED_READ | AW4_MOMENT_READ_RAW_SCALE | AW4_MOMENT_FRESH_PROXY |
                                 AW4_MOMENT_PENDING),
              "run-time flag marker collides with a moment flag");
constexpr int mspec(int kind, int flags = 0) { return kind | (flags << 4); }
constexpr int kind_of(int spec) { return spec & 15; }
constexpr int flags_of(int spec) { return spec >> 4; }
// The flags that change what a kind computes (round-to-nearest: EDEN; the zero floor of
// round-to-nearest lives in its lookup table).
constexpr int spec_flags_mask(int kind) {
    return kind == K_FP32 ? 0
         : kind == K_RTN ? AW4_MOMENT_EDEN
         : kind == K_USR ? (AW4_MOMENT_EDEN | AW4_MOMENT_GUARDS | AW4_MOMENT_ZERO_FLOOR | AW4_MOMENT_SAMPLED_READ |
                            AW4_MOMENT_READ_RAW_SCALE)
         : kind == K_LA  ? AW4_MOMENT_PENDING  // a pending lookahead m2 keeps fp32 values, no codes
                         : (AW4_MOMENT_EDEN | AW4_MOMENT_GUARDS | AW4_MOMENT_ZERO_FLOOR);
}

// A lookahead m2 spec marked pending: fp32 values, sampled before the update, no codes.
constexpr bool pending_spec(int spec) { return kind_of(spec) == K_LA && (flags_of(spec) & AW4_MOMENT_PENDING) != 0; }

// Lookup-table ids (aw4_encode_tables): round-to-nearest tables, then level-count tables.
constexpr int kLutRtn[AW4_NUM_CODEBOOKS] = {0, 1, 2, 3, 4};
constexpr int kLutRtnDyn4Floor = 5;
constexpr int kLutLevels[AW4_NUM_CODEBOOKS] = {6, 7, 8, 9, 10};

// Bucket of x -> code = base + (x >= thr); lv_lo / lv_hi are cb[min(code, 15)] of the two
// outcomes: the code's level in round-to-nearest tables (what EDEN multiplies by), the
// upper neighbour b of x in level-count tables.
struct __align__(16) LutEntry {
    float thr;
    uint32_t base;
    float lv_lo;
    float lv_hi;
};

// Neighbouring levels of a searchsorted-left index (_compiled_quantization.py:30-38).
struct __align__(16) PairEntry {
    float a;          // cb[lo]
    float b;          // cb[hi]
    float width_rcp;  // RN(1 / max(b - a, 1e-12))
    uint32_t lohi;    // lo | hi << 8
};

// Per-block update-SR quantities for each searchsorted index i (update_sr_tables()), with
// c = sqrt(s / bias) the block's scale factor and E(l) = c * sqrt(l) + eps for a level l, so that
// the preconditioner of l is 1 / E(l) (_compiled_quantization.py:83-85).
struct __align__(8) UpdEntry {
    float sqrt_hi;  // sqrt(b), b the upper level of the interval
    float g;        // (sqrt(b) - sqrt(a)) * 2^-24 / E(a), a the lower level (0: no interval)
};

// The level-only part of the update-SR quantities of a searchsorted index i, with a = cb[lo],
// b = cb[hi] its levels (host-computed in double, each rounded once to fp32).
struct __align__(16) UsrPair {
    float sqrt_lo;  // RN(sqrt(a)), 0 for a <= 0
    float sqrt_hi;  // RN(sqrt(b)), 0 for b <= 0
    float gap_s;    // RN(sqrt(b) - sqrt(a)) * 2^-24 (exact), 0 unless b > a >= 0
    float b_gt_a;   // 1 where b > a (fp32 levels), else 0
};

// All tables of all codebooks, built on the host and kept in device memory.
struct Tables {
    float codebook[AW4_NUM_CODEBOOKS][16];
    UsrPair usr[AW4_NUM_CODEBOOKS][kPairs];  // per searchsorted index (update-SR)
    PairEntry pairs[AW4_NUM_CODEBOOKS][kPairs];
    float2 dec[AW4_NUM_CODEBOOKS][256];  // code byte -> (level of low nibble, level of high nibble)
    LutEntry lut[AW4_NUM_LUTS][AW4_LUT_ENTRIES];
};

// LDS views of the tables one moment needs.
struct MomentTables {
    const float* cb;
    const PairEntry* pairs;
    const float2* dec;
    const LutEntry* lut;
    const UsrPair* usr;
};

// LDS scratch of one block's encode: update-SR tables of the block and the staging area
// of its 64 code bytes (written a quarter at a time, stored to memory in one piece).
struct BlockScratch {
    UpdEntry* upd;      // kPairs entries (update-SR only)
    float* pre;         // the reference's preconditioners of the 16 levels (usr_level_preconds)
    uint16_t* stage;    // 32 code words: word 8q + j is lane j's word of quarter q
};

// Code bytes of one wave tile: 8 blocks of 64; bytes of its 16-bit values: 8 blocks of 256.
constexpr int kWaveCodeBytes = kBlocksPerWave * kBlock / 2;
constexpr int kWaveImageBytes = kBlocksPerWave * kBlock * 2;

// LDS scratch of one wave (8 blocks).  In kernels that move tiles through LDS, its first
// kWaveImageBytes bytes also pass the loaded code words of both moments to their lanes before a
// tile's update, and then hold the updated 16-bit parameters until they are stored.
struct WaveScratch {
    UpdEntry upd[kBlocksPerWave][kPairs];
    float pre[kBlocksPerWave][16];
    uint16_t stage[kBlocksPerWave][32];

    __device__ BlockScratch block(int grp) { return BlockScratch{upd[grp], pre[grp], stage[grp]}; }
    __device__ uint8_t* code_words() { return (uint8_t*)&upd[0][0]; }
};
static_assert(sizeof(WaveScratch::upd) >= 2 * kWaveCodeBytes, "code words of two moments in the update-SR tables");
static_assert(sizeof(WaveScratch) >= kWaveImageBytes, "a tile's 16-bit parameters in the wave's scratch");

// Exponent and top 3 mantissa bits of x, clamped to the table's range (one med3).
__device__ __forceinline__ int lut_field(uint32_t u) {
    return min(max((int)__builtin_amdgcn_ubfe(u, 20, 11), AW4_LUT_EXP0 - 1), AW4_LUT_EXP0 - 2 + AW4_LUT_HALF);
}

// Bucket of an x >= -0 (second moments): only the magnitude half of the table.
__device__ __forceinline__ int lut_bucket_unsigned(float x) { return lut_field(f2u(x)) - (AW4_LUT_EXP0 - 1); }

__device__ __forceinline__ int lut_bucket_signed(float x) {
    const uint32_t u = f2u(x);
    return lut_field(u) - (AW4_LUT_EXP0 - 1) + (int)(u >> 31) * AW4_LUT_HALF;
}

// Decode the 4 values of one 16-bit code word: two LDS reads of level pairs.
__device__ __forceinline__ void decode4(const float2* dec, uint32_t w, float scale, float (&m)[4]) {
    const float2 lo = dec[w & 0xffu];
    const float2 hi = dec[(w >> 8) & 0xffu];
    m[0] = lo.x * scale;
    m[1] = lo.y * scale;
    m[2] = hi.x * scale;
    m[3] = hi.y * scale;
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Update-SR (_compiled_quantization.py:74-109) decides lower with probability
//   P = (f(x) - f(b)) / (f(a) - f(b)),  f(l) = 1 / (sqrt((s * l) / bias) + eps),
// for the levels a < x <= b around x.  With c = sqrt(s / bias) and E(l) = c * sqrt(l) + eps,
// f(l) = 1 / E(l) and, exactly,
//   P = E(a) * (sqrt(b) - sqrt(x)) / ((sqrt(b) - sqrt(a)) * E(x)),
// so u < P exactly when
//   Q = (sqrt(b) - sqrt(x)) - u * ((sqrt(b) - sqrt(a)) / E(a)) * E(x) > 0:
// one square root and no division per value.  The reference rounds each of its steps in fp32
// (its f values within 5 ulps with a faithful square root, then a difference and a quotient),
// and Q here is rounded too; the two decisions provably agree when
//   |Q| > 2^-19 * (E(b) / c + sqrt(b))
// (32 units of 2^-24: the bound, first order in 2^-24, is 20.05 units times E(b) / c for the
// reference's rounding and 24.01 units times sqrt(b) for Q's).  The band is taken per value as
// 2^-18 * sqrt(b) + 2^-19 * eps / c (E(b) / c = sqrt(b) + eps / c; the computed band is within a
// few ulps of that, far inside the slack of 32 units against 20.05 and 24.01): most values sit
// on the small levels of their block, where it is several times narrower than the bound for
// b = 1.  Values inside it (about 1 in 10^5 on heavy-tailed second moments) take usr_exact,
// the reference's own operations.  The interval is valid when b > a
// and fp32 f(a) > f(b); the latter is certain when c * (sqrt(b) - sqrt(a)) > 2^-20 * E(b) (the
// true relative gap of f(a) and f(b) against their 5-ulp rounding); a block where it is not
// (c tiny against eps) decides every value with usr_exact.
constexpr float kUsrBand = 0x1p-19f;

struct UsrBlock {
    float c;      // sqrt(s / bias), within 3 ulps
    float band0;  // the block's part of the band, 2^-19 * eps / c (+inf: decide every value exactly)
};

// The block's 17 UpdEntry of the searchsorted indices (two per lane), each from its own level pair:
// E(a) and E(b) are formed where they are used, so no lane reads another's.
__device__ __forceinline__ UsrBlock update_sr_tables(const MomentTables& L, int j, float s, const aw4_moment& M,
                                                     UpdEntry* upd) {
    const float c = sqrt_faithful(s * M.sr_bias_rcp);
    const float c_rcp = rcp_faithful(c);
    // Entries 1..16 in two rounds of the block's 8 lanes; entry 0 (no level below x) has
    // lo == hi and no interval.
    bool certain = true;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int i = 1 + j + 8 * h;
        const UsrPair up = L.usr[i];
        const float e_lo = __builtin_fmaf(c, up.sqrt_lo, M.sr_eps), e_hi = __builtin_fmaf(c, up.sqrt_hi, M.sr_eps);
        // over the real intervals: c * gap > 2^-20 * E(b), both sides scaled by 2^-24, which leaves the
        // comparison exact: with c >= 1e-6, every codebook's real gaps >= 2^-6 and its positive levels
        // >= 2^-9, both products of a real interval stay far above the subnormals
        certain = certain & ((up.b_gt_a == 0.0f) | (c * up.gap_s > 0x1p-44f * e_hi));
        // E(a) = 0 (a = 0 with eps = 0): f(a) is infinite and P = 0, so g = +inf decides upper
        // (a draw of exactly 0 gives Q = NaN, which counts as sure and decides upper too)
        const float g = e_lo > 0.0f ? up.gap_s * rcp_faithful(e_lo) : __builtin_inff();
        upd[i] = UpdEntry{up.sqrt_hi, g};
    }
    // Entry 0: no level below x (x = 0 for dyn4), where the code does not depend on the draw:
    // Q = NaN marks the value sure in every block, certain or not (an all-zero block's scale is
    // the 1e-12 floor, which no band covers).
    if (j == 0) upd[0] = UpdEntry{__builtin_nanf(""), 0.0f};
    // every interval of the block certain (its 8 lanes, 16 entries)
    uint32_t all = certain ? 1u : 0u;
    all = min(all, dpp_u32<kQuadXor1>(all));
    all = min(all, dpp_u32<kQuadXor2>(all));
    all = min(all, dpp_u32<kHalfRowMirror>(all));
    wave_lds_sync();
    const float band0 = kUsrBand * (M.sr_eps * c_rcp);
    return UsrBlock{c, all ? band0 : __builtin_inff()};
}

// Uniforms of this lane's 4 values of quarter q in its block (block blk0 + grp of one write
// of moment M), scaled by 2^24: U = u * 2^24 is exact for every float u, and an integer in
// [0, 2^24) for the generator's 24-bit draws.  On-device draws: the block's values are
// stream positions rng_offset + 128 * block + 32 q + 4 j + t (rng_offset a multiple of
// 128), so the lane's 16 uniforms come from the three Philox calls of position group
// rng_offset / 128 + block; call r is made at quarter r, into words 4r .. 4r+3 of `rw`, and
// quarter q reads words 3q .. 3q+2.  The loop over q must be unrolled (constant indices).
__device__ __forceinline__ void draws_quarter(const aw4_moment& M, int64_t blk0, int grp, int j, int q, bool active,
                                              uint32_t (&rw)[12], float (&u)[4]) {
    if (__builtin_expect((M.flags & AW4_MOMENT_EXT_DRAWS) != 0, 0)) {
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (active)
            v = *(gptr<const f32x4>)(gaddr<const float>(M.draws) + (blk0 + grp) * kBlock + 32 * q + 4 * j);
        u[0] = v.x * 0x1p24f; u[1] = v.y * 0x1p24f; u[2] = v.z * 0x1p24f; u[3] = v.w * 0x1p24f;
    } else {
        if (q < 3) philox_tile_call(M.rng_seed, (M.rng_offset >> 7) + (uint64_t)blk0, grp, j, q, &rw[4 * q]);
        lane_fields4(&rw[3 * q], u);
    }
}

// The reference's preconditioner of a level or value l: fp32(1 / (sqrt(max((s * l) / bias, 0))
// + eps)), each operation correctly rounded (ATen's division, 1.0 / t as a reciprocal) and the
// square root correctly rounded (ATen's is within an ulp of it).
__device__ __forceinline__ float usr_precond(const aw4_moment& M, float s, float l) {
    const float v = clamp_min_nan((s * l) / M.sr_bias, 0.0f);
    return 1.0f / (sqrt_cr(v) + M.sr_eps);
}

// Update-SR decision by the reference's operations (_compiled_quantization.py:74-109):
// valid = (b > a) & (f(a) - f(b) > 0); lower = u < (f(x) - f(b)) / max(f(a) - f(b), 1e-30),
// u = U * 2^-24.  The clamp of P to [0, 1] never changes u < P for u in [0, 1).  fa and fb are
// the preconditioners of the levels a and b (usr_precond of the block's scale and the level,
// from the block's table: usr_level_preconds).
__device__ __forceinline__ void usr_exact(const aw4_moment& M, float s, float x, float a, float b, float fa, float fb,
                                          float U, bool& valid, bool& lower) {
    const float fx = usr_precond(M, s, x);
    const float den = fa - fb;
    valid = (b > a) & (den > 0.0f);
    lower = U * 0x1p-24f < (fx - fb) / clamp_min_nan(den, 1e-30f);
}

// The reference's preconditioners of the block's 16 levels, f(l) = usr_precond(s, l), into the
// block's 16-entry table (two per lane), for usr_exact: the same function of the same inputs as
// an evaluation per value, so the same bits.  Built only in a block encode where some quarter
// needs the exact form.
__device__ __forceinline__ void usr_level_preconds(const MomentTables& L, int j, float s, const aw4_moment& M,
                                                   float* pre) {
#pragma unroll
    for (int h = 0; h < 2; ++h) pre[j + 8 * h] = usr_precond(M, s, L.cb[j + 8 * h]);
    wave_lds_sync();
}

// The quick decision (see update_sr_tables): returns Q, where Q > 0 means lower; `sure` is false
// inside the value's band 2^-18 * sqrt(b) + band0.  U = u * 2^24.
__device__ __forceinline__ float usr_quick(const UpdEntry& ue, const UsrBlock& ub, float eps, float x, float U,
                                           bool& sure) {
    const float w = sqrt_faithful(x);
    const float ex = __builtin_fmaf(ub.c, w, eps);
    const float q = __builtin_fmaf(-U, ue.g * ex, ue.sqrt_hi - w);
    // NaN: sure (entry 0, whose sqrt_hi is NaN, or a zero draw with g = +inf)
    sure = !(__builtin_fabsf(q) <= __builtin_fmaf(ue.sqrt_hi, 2.0f * kUsrBand, ub.band0));
    return q;
}

// NaN-propagating max(acc, |v|): v_maximum3_f32 with |.| operands.
__device__ __forceinline__ float abs_max_acc(float acc, float v) {
    return __builtin_elementwise_maximum(acc, __builtin_fabsf(v));
}

// The 16 values of this lane that a block encode reads, a quarter (4 values) at a time:
// held in registers, or staged in LDS by the code that produced them (which also kept
// their running max |v|), so that they occupy no registers until their quarter is encoded.
struct RegValues {
    const float (&m)[16];
    __device__ float abs_max() const {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) a = abs_max_acc(a, m[i]);
        return a;
    }
    __device__ void quarter(int q, float (&v)[4]) const {
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = m[4 * q + t];
    }
};
struct StagedValues {
    const f32x4* lane_q0;  // this lane's quarter 0; quarter q is 64 entries further
    float amax;            // max |v| over the 16 values (NaN-propagating)
    __device__ float abs_max() const { return amax; }
    __device__ void quarter(int q, float (&v)[4]) const {
        const f32x4 x = lane_q0[64 * q];
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
    }
};

// The scales a block encode produced: s = max(absmax, 1e-12) (every lane) and the stored
// scale (s, or its EDEN calibration; valid in lane j == 0).
struct BlockScales {
    float raw;
    float stored;
};

template <int SPEC, bool kNonNeg, class Values>
__device__ __forceinline__ BlockScales encode_block(const aw4_moment& M, const MomentTables& L, int64_t blk0, int grp,
                                                    int j, bool active, const Values& vals, BlockScratch sc) {
    // max |m| over the lane's values, then over the block's 8 lanes on the bit patterns
    // (non-negative floats and NaNs order as unsigned integers).
    const uint32_t amax = block_max_u32(f2u(vals.abs_max()));
    const float s = u2f(max(amax, 0x2B8CBCCCu));  // max(absmax, fp32(1e-12))
    bool fast = s < 0x1p125f;                      // otherwise huge, infinite or NaN: IEEE division
    const float y = div_cr(1.0f, s);               // RN(1 / s): normal on the fast path
    constexpr int KIND = kind_of(SPEC), MF = flags_of(SPEC);
    constexpr bool kDyn = (MF & kFlagsAtRunTime) != 0;
    const int flags = kDyn ? M.flags : MF;
    const bool eden = (flags & AW4_MOMENT_EDEN) != 0;
    const bool guards = (flags & AW4_MOMENT_GUARDS) != 0;
    const bool floor0 = (flags & AW4_MOMENT_ZERO_FLOOR) != 0;
    UsrBlock ub{0.0f, 0.0f};
    if constexpr (KIND == K_USR) {
        ub = update_sr_tables(L, j, s, M, sc.upd);
        fast = fast && s * M.sr_bias_rcp < 0x1p127f;  // (s * x) / bias stays far from overflow
    }
    // One branch for the whole wave: the IEEE forms are exact for every block, so a wave
    // with any huge, infinite or NaN scale runs them for all of its blocks, and the common
    // case is a scalar branch instead of a divergent one.
    const bool wave_fast = __builtin_amdgcn_ballot_w64(!fast) == 0;
    wave_lds_sync();  // the stage's previous contents have been read

    float acc_xx[4] = {0.0f, 0.0f, 0.0f, 0.0f}, acc_xl[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    uint32_t rw[12];  // Philox words of this lane's position group (stochastic kinds)
    bool level_preconds = false;  // the block's table of level preconditioners is built (update-SR)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float x[4], mq[4];
        vals.quarter(q, mq);
        if (__builtin_expect(wave_fast, 1)) {
#pragma unroll
            for (int t = 0; t < 4; ++t) x[t] = div_by_rcp(mq[t], s, y);
        } else {
            // torch.searchsorted orders NaN above every level.  A NaN x (only in blocks whose
            // scale is not finite, which all take this path) becomes the positive quiet NaN, so
            // the signed lookup, which reads the sign bit, puts it in the top bucket too.
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float v = mq[t] / s;
                x[t] = v != v ? __builtin_nanf("") : v;
            }
        }
        uint32_t code[4];
        float lv[4];
        if constexpr (KIND == K_RTN) {
            // code = base + (x >= thr); the level for EDEN comes with the entry.
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const LutEntry e = L.lut[kNonNeg ? lut_bucket_unsigned(x[t]) : lut_bucket_signed(x[t])];
                const bool up = x[t] >= e.thr;
                code[t] = e.base + (up ? 1u : 0u);
                lv[t] = up ? e.lv_hi : e.lv_lo;
            }
        } else {
            float u[4];  // the uniforms times 2^24
            draws_quarter(M, blk0, grp, j, q, active, rw, u);
            // Both rules pick level lo = max(idx - 1, 0) or hi = min(idx, 15), idx = number of levels
            // below x.  Since u is in [0, 1), u < clamp(P, 0, 1) == u < P for every P (NaN included),
            // so the clamps of the reference never change a code and the guards become masks.
            int idx[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const LutEntry le = L.lut[kNonNeg ? lut_bucket_unsigned(x[t]) : lut_bucket_signed(x[t])];
                idx[t] = (int)le.base + (x[t] >= le.thr ? 1 : 0);
            }
            if constexpr (KIND == K_SSR) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    // P(hi) = (x - a) / max(b - a, 1e-12), 0 where b == a (there lo == hi); guards
                    // x <= a -> lo, x >= b -> hi (_compiled_quantization.py:60-71).
                    const PairEntry pe = L.pairs[idx[t]];
                    const float width = pe.b - pe.a;
                    const float p = div_by_rcp(x[t] - pe.a, width < 1e-12f ? 1e-12f : width, pe.width_rcp);
                    bool upper = u[t] < p * 0x1p24f;
                    if (guards) upper = (upper | (x[t] >= pe.b)) & !(x[t] <= pe.a);
                    code[t] = (uint32_t)min(max(idx[t] - (upper ? 0 : 1), 0), 15);
                }
            } else {
                // P(lo) = (f(x) - f(b)) / max(f(a) - f(b), 1e-30), 1 on invalid intervals
                // (_compiled_quantization.py:74-109).  On a valid interval P is 0 at x == b, so
                // x >= b picks hi with or without the guards; the guards let x >= b override an
                // invalid interval, and add x <= a -> lo, which holds exactly when no level is
                // below x (idx == 0), where lo and hi are both code 0: that guard changes no code
                // (nor the level EDEN reads) and is not evaluated.
                // the decision as a float whose sign is the outcome (> 0: lower), so that the two
                // paths below meet in plain registers
                float dq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                uint64_t unsure = 1;  // lanes (bits) with a value the quick test leaves open
                bool open[4] = {true, true, true, true};  // per value: left open (every value off the quick path)
                if (__builtin_expect(wave_fast, 1)) {
                    unsure = 0;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const UpdEntry ue = sc.upd[idx[t]];
                        bool sure;
                        dq[t] = usr_quick(ue, ub, M.sr_eps, x[t], u[t], sure);
                        open[t] = !sure;
                        unsure |= __builtin_amdgcn_ballot_w64(!sure);
                    }
                }
                // A quarter with any open value (a few in a hundred) decides its open values again
                // by the reference's operations (a branch per value slot, taken where any lane has
                // that slot open; the quarter's branch is uniform).  Where the quick test was sure
                // the two agree.  It leaves code = idx - lower with idx in [0, 15], the clamps folded
                // into lower and idx.
                if (__builtin_expect(unsure != 0, 0)) {  // laid out after the loop (cold)
                    // the levels' preconditioners once per block encode, when a quarter first needs them
                    if (!level_preconds) {
                        usr_level_preconds(L, j, s, M, sc.pre);
                        level_preconds = true;
                    }
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        if (!open[t]) continue;
                        const PairEntry pe = L.pairs[idx[t]];
                        bool valid, dl;
                        usr_exact(M, s, x[t], pe.a, pe.b, sc.pre[pe.lohi & 0xffu], sc.pre[pe.lohi >> 8], u[t], valid,
                                  dl);
                        // bitwise operators: the operands are all computed, and short-circuit
                        // forms become per-value branches
                        const bool at_b = x[t] >= pe.b;
                        const bool ok = valid & (idx[t] > 0);
                        const bool lower = guards ? ((!ok) | dl) & !at_b : (!ok) | (dl & !at_b);
                        // idx 0: code 0; idx 16: code 15
                        dq[t] = (lower & ((uint32_t)(idx[t] - 1) < 15u)) ? 1.0f : -1.0f;
                        idx[t] = min(idx[t], 15);
                    }
                }
                // Where the quick test decided every value of the quarter: code = idx - lower,
                // without guards or clamps.  The block is certain, so every interval is valid.  No
                // level below x (idx = 0): Q is NaN and lower false, code 0.  x at its upper level
                // b (where both forms of the rule pick hi): Q = (sqrt(b) - w) - u * g * E(b) with w
                // within an ulp of sqrt(b), so a sure Q is negative and lower false.  idx <= 15,
                // as x <= 1, the top level of the update-SR codebooks, on the quick path.
#pragma unroll
                for (int t = 0; t < 4; ++t) code[t] = (uint32_t)(idx[t] - (dq[t] > 0.0f ? 1 : 0));
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if (floor0) code[t] = max(code[t], 1u);
                lv[t] = eden ? L.cb[code[t]] : 0.0f;
            }
        }
        if (eden) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                acc_xx[t] = acc_xx[t] + x[t] * x[t];
                acc_xl[t] = acc_xl[t] + x[t] * lv[t];
            }
        }
        sc.stage[8 * q + j] = (uint16_t)(code[0] | (code[1] << 4) | (code[2] << 8) | (code[3] << 12));
    }
    wave_lds_sync();
    if (active) {
        // lane j: code bytes 8j .. 8j+7 of its block; the tile's codes start at byte blk0 * 64
        const u32x2 w = *(const u32x2*)(sc.stage + 4 * j);
        const gptr<uint8_t> codes = gaddr<uint8_t>(M.codes) + blk0 * (kBlock / 2);
        __builtin_nontemporal_store(w, (gptr<u32x2>)(codes + (uint32_t)(grp * (kBlock / 2) + 8 * j)));
    }

    float scale = s;
    if (eden) {
        // s' = s * (sum x*x / max(sum x*cb[code], 1e-12))  (_optimized_quantization.py:81-85)
        const float num = block_sum_cross(acc_xx);
        const float den = block_sum_cross(acc_xl);
        scale = s * div_cr(num, clamp_min_nan(den, 1e-12f));  // num in [1, 128]: a normal quotient
    }
    if (active && j == 0) __builtin_nontemporal_store(scale, gaddr<float>(M.scales) + blk0 + grp);
    return BlockScales{s, scale};
}

// ---------------------------------------------------------------------------
// Lookahead update-SR (quantize_dyn4_la_upd_sr, quantization.py:779-895), in float64 as
// the reference computes it: for levels a <= x <= b of the block-scaled value
// x = clamp(z / s, 0, 1), with q = s * level and the next step's second moment
// n(q) = max(beta2 * q + fresh, 0),
//   P(lo) = (f(n(z)) - f(n(q_hi))) / max(f(n(q_lo)) - f(n(q_hi)), 1e-300),
//   f(n) = 1 / (sqrt(n / bias) + eps),
// replaced by 1 - clamp((z - q_lo) / max(q_hi - q_lo, 1e-300), 0, 1) where the interval is
// flat (|f(n(q_lo)) - f(n(q_hi))| <= 1e-12 max(|f(n(q_lo))|, |f(n(q_hi))|, 1)), 1 where it is
// degenerate (q_hi <= q_lo), clamped to [0, 1].  No guards: z at a level gives 0 or 1
// through the formula itself.
// ---------------------------------------------------------------------------

__device__ __forceinline__ double clamp_min0_nan(double v) { return v < 0.0 ? 0.0 : v; }
__device__ __forceinline__ double clamp01_nan_d(double v) { return v < 0.0 ? 0.0 : (v > 1.0 ? 1.0 : v); }
__device__ __forceinline__ double max_nan(double a, double b) { return (a != a || b != b) ? a + b : (a > b ? a : b); }

__device__ __forceinline__ double la_prob_lo(const aw4_moment& M, float z, float a, float b, float s, double fresh) {
    const double s64 = (double)s, z64 = (double)z;
    const double q_lo = s64 * (double)a, q_hi = s64 * (double)b;  // exact: products of two floats
    const double beta2 = M.la_beta2;
    const double n_lo = clamp_min0_nan(beta2 * q_lo + fresh);
    const double n_ref = clamp_min0_nan(beta2 * z64 + fresh);
    const double n_hi = clamp_min0_nan(beta2 * q_hi + fresh);
    const double p_lo = 1.0 / (sqrt(n_lo / M.la_bias) + M.la_eps);
    const double p_ref = 1.0 / (sqrt(n_ref / M.la_bias) + M.la_eps);
    const double p_hi = 1.0 / (sqrt(n_hi / M.la_bias) + M.la_eps);
    const double denom = p_lo - p_hi, width = q_hi - q_lo;
    const double raw = (p_ref - p_hi) / (denom < 1e-300 ? 1e-300 : denom);
    const double fallback = 1.0 - clamp01_nan_d((z64 - q_lo) / (width < 1e-300 ? 1e-300 : width));
    const bool degenerate = width <= 0.0;
    double flat_scale = max_nan(fabs(p_lo), fabs(p_hi));
    flat_scale = flat_scale < 1.0 ? 1.0 : flat_scale;
    const bool flat = !degenerate && fabs(denom) <= 1e-12 * flat_scale;
    double p = flat ? fallback : raw;
    if (degenerate) p = 1.0;
    return clamp01_nan_d(p);
}

// Float64 uniforms of this lane's 4 values of quarter q (see draws_quarter): the
// generator's 24-bit fields times 2^-24 (U: the fields themselves), or a caller's doubles
// (AW4_MOMENT_EXT_DRAWS; U unused).
__device__ __forceinline__ void la_draws_quarter(const aw4_moment& M, int64_t blk0, int grp, int j, int q, bool active,
                                                 uint32_t (&rw)[12], double (&u)[4], float (&U)[4]) {
    if (M.flags & AW4_MOMENT_EXT_DRAWS) {
        const gptr<const double> d = gaddr<const double>(M.draws) + (blk0 + grp) * kBlock + 32 * q + 4 * j;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            u[t] = active ? d[t] : 0.0;
            U[t] = 0.0f;
        }
    } else {
        if (q < 3) philox_tile_call(M.rng_seed, (M.rng_offset >> 7) + (uint64_t)blk0, grp, j, q, &rw[4 * q]);
        lane_fields4(&rw[3 * q], U);
#pragma unroll
        for (int t = 0; t < 4; ++t) u[t] = (double)U[t] * 0x1p-24;
    }
}

// Quick lookahead decision in fp32.  With r = sqrt(n), E = r / sqrt(bias) + eps, the rule's
// P = (p(z) - p(q_hi)) / (p(q_lo) - p(q_hi)) is exactly N / D with
//   N = (q_hi - z) (r_hi + r_lo) E_lo,  D = (q_hi - q_lo) (r_hi + r_z) E_z,
// positive factors without cancellation, which fp32 evaluates within about 2^-19 each.  The
// decision u < P is taken without a division as the sign of T = u D - N (one fused rounding),
// within about 2^-17.9 max(N, D) of D (u - P).  The reference's float64 P itself is off by a
// few 2^-53 M, where M = max(p_lo, 1) / (p_lo - p_hi) and
//   M D = (r_hi + r_lo) E_hi max(E_lo, 1) (r_hi + r_z) E_z sqrt(bias) / beta2
// (the interval width cancels).  The decision is sure outside the band
// |T| > 2^-16 max(N, D) + 2^-46 M D (that is, |u - P| > 2^-16 max(P, 1) + 2^-46 M); values
// inside it, or with M >= 2^36 (near the reference's switch to its value-linear form at 1e12),
// or with n_lo below 2^-100 (where fp32 loses the small terms, and where p_lo = +inf makes the
// reference's flat test true) take la_prob_lo.  rb = 1 / sqrt(bias) and sb = sqrt(bias) / beta2
// within a few ulps; fresh within 3 ulps of the reference's float64 term.
struct LaQuick {
    float beta2, rb, eps, sb;
};
__device__ __forceinline__ void la_quick(const LaQuick& k, float z, float a, float b, float s, float fresh, float U,
                                         bool& lower, bool& sure) {
    const float q_lo = s * a, q_hi = s * b;
    const float n_lo = __builtin_fmaf(k.beta2, q_lo, fresh);
    const float n_hi = __builtin_fmaf(k.beta2, q_hi, fresh);
    const float n_z = __builtin_fmaf(k.beta2, z, fresh);
    const float r_lo = sqrt_faithful(n_lo), r_hi = sqrt_faithful(n_hi), r_z = sqrt_faithful(n_z);
    const float e_lo = __builtin_fmaf(r_lo, k.rb, k.eps);
    const float e_hi = __builtin_fmaf(r_hi, k.rb, k.eps);
    const float e_z = __builtin_fmaf(r_z, k.rb, k.eps);
    const float d_hi = __builtin_fmaf(s, b, -z);
    const float w = s * (b - a);
    const float s_lo = r_hi + r_lo, sz_ez = (r_hi + r_z) * e_z;
    const float num = (d_hi * s_lo) * e_lo;
    const float den = w * sz_ez;
    const float md = (((s_lo * e_hi) * __builtin_fmaxf(e_lo, 1.0f)) * sz_ez) * k.sb;
    const float u = U * 0x1p-24f;
    const float t = __builtin_fmaf(u, den, -num);
    const float band = __builtin_fmaf(0x1p-16f, __builtin_fmaxf(num, den), 0x1p-46f * md);
    lower = t < 0.0f;
    // comparisons with NaN are false: a NaN N, D or M D is never sure; D = 0 (M infinite) neither
    sure = (__builtin_fabsf(t) > band) & (md < 0x1p36f * den) & (n_lo >= 0x1p-100f);
}

// Lookahead update-SR of this lane's 16 values z of block blk0 + grp (clamped at 0 first).
// fresh: (1-beta2) * g^2 in float64 from the gradients g, or with AW4_MOMENT_FRESH_PROXY
// fp32(w2f * z) (the v-proxy's (1 - beta2) * m2, fp32(1-beta2) = w2f).  Stores the codes
// and scale (store), and/or returns each value's sample fp32(s * level) (sampled).
__device__ __forceinline__ BlockScales encode_block_la(const aw4_moment& M, const MomentTables& L, int64_t blk0,
                                                       int grp, int j, bool active, const float (&z_in)[16],
                                                       const float (&g)[16], float w2f, bool store, float* sampled,
                                                       BlockScratch sc) {
    float z[16];
    float amf = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        z[i] = clamp_min_nan(z_in[i], 0.0f);
        amf = abs_max_acc(amf, z[i]);
    }
    const uint32_t amax = block_max_u32(f2u(amf));
    const float s = u2f(max(amax, 0x2B8CBCCCu));  // max(absmax, fp32(1e-12))
    const bool wave_fast = __builtin_amdgcn_ballot_w64(!(s < 0x1p125f)) == 0;
    const float y = div_cr(1.0f, s);
    const bool proxy = (M.flags & AW4_MOMENT_FRESH_PROXY) != 0;
    // the quick form needs the generator's 24-bit draws and finite, normal block scales
    const bool quick = wave_fast & ((M.flags & AW4_MOMENT_EXT_DRAWS) == 0);
    const float sqrt_bias = sqrt_faithful((float)M.la_bias);
    const LaQuick lq{(float)M.la_beta2, rcp_faithful(sqrt_bias), (float)M.la_eps,
                     sqrt_bias * rcp_faithful((float)M.la_beta2)};
    const float wf = (float)M.la_fresh_weight;
    uint32_t rw[12];
    wave_lds_sync();  // the stage's previous contents have been read
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        double u[4];
        float U[4];
        la_draws_quarter(M, blk0, grp, j, q, active, rw, u, U);
        uint32_t code[4];
        int idx[4];
        float a[4], b[4];
        bool lower[4];
        uint64_t unsure = quick ? 0 : ~0ull;  // lanes (bits) with a value the quick form leaves open
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int i = 4 * q + t;
            const float xq = __builtin_expect(wave_fast, 1) ? div_by_rcp(z[i], s, y) : z[i] / s;
            const float x = clamp01_nan(xq);
            const LutEntry le = L.lut[lut_bucket_unsigned(x)];
            const bool up = x >= le.thr;
            idx[t] = (int)le.base + (up ? 1 : 0);
            b[t] = up ? le.lv_hi : le.lv_lo;   // cb[min(idx, 15)]
            a[t] = L.cb[idx[t] > 0 ? idx[t] - 1 : 0];
            if (quick) {
                const float fresh = proxy ? clamp_min_nan(w2f * z_in[i], 0.0f) : (wf * g[i]) * g[i];
                bool sure;
                la_quick(lq, z[i], a[t], b[t], s, fresh, U[t], lower[t], sure);
                // idx == 0 (z = 0): a degenerate interval, P = 1, and lo == hi
                unsure |= __builtin_amdgcn_ballot_w64(!(sure | (idx[t] == 0)));
            }
        }
        // A quarter with any open value is decided again by the reference's float64 rule, every
        // value of it (where the quick form was sure the two agree).  The branch is uniform.
        if (unsure != 0) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int i = 4 * q + t;
                const double fresh = proxy ? (double)clamp_min_nan(w2f * z_in[i], 0.0f)
                                           : M.la_fresh_weight * ((double)g[i] * (double)g[i]);
                lower[t] = u[t] < la_prob_lo(M, z[i], a[t], b[t], s, fresh);
            }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int i = 4 * q + t;
            code[t] = (uint32_t)min(max(idx[t] - (lower[t] ? 1 : 0), 0), 15);
            if (sampled) sampled[i] = s * (lower[t] ? a[t] : b[t]);
        }
        if (store) sc.stage[8 * q + j] = (uint16_t)(code[0] | (code[1] << 4) | (code[2] << 8) | (code[3] << 12));
    }
    if (store) {
        wave_lds_sync();
        if (active) {
            const u32x2 w = *(const u32x2*)(sc.stage + 4 * j);
            const gptr<uint8_t> codes = gaddr<uint8_t>(M.codes) + blk0 * (kBlock / 2);
            __builtin_nontemporal_store(w, (gptr<u32x2>)(codes + (uint32_t)(grp * (kBlock / 2) + 8 * j)));
        }
        if (active && j == 0) __builtin_nontemporal_store(s, gaddr<float>(M.scales) + blk0 + grp);
    }
    return BlockScales{s, s};
}

// Runtime dispatch over the rounding kind (generic kernels).
template <bool kNonNeg, class Values>
__device__ __forceinline__ BlockScales encode_block_any(const aw4_moment& M, const MomentTables& L, int64_t blk0,
                                                        int grp, int j, bool active, const Values& v, BlockScratch sc) {
    if (M.rounding == K_RTN)
        return encode_block<mspec(K_RTN, kFlagsAtRunTime), kNonNeg>(M, L, blk0, grp, j, active, v, sc);
    if (M.rounding == K_SSR)
        return encode_block<mspec(K_SSR, kFlagsAtRunTime), kNonNeg>(M, L, blk0, grp, j, active, v, sc);
    return encode_block<mspec(K_USR, kFlagsAtRunTime), kNonNeg>(M, L, blk0, grp, j, active, v, sc);
}

}  // namespace aw4
