// The fused AdamW step over one launch table: per-tile pipeline (prefetch the next
// tile's inputs, decode, AdamW, re-encode, store) specialised by moment kinds and
// parameter dtype.
#pragma once

#include <type_traits>

#include "aw4_codec.h"

namespace aw4 {

constexpr int kWaveTile = kBlock * kBlocksPerWave;  // 1024 values per wave tile
constexpr int kTilesPerWave = 4;                    // consecutive wave tiles one wave processes
constexpr int kThreads = 256;
constexpr int kWavesPerGroup = kThreads / 64;

// Parameter/gradient storage kinds (AW4_F32 / AW4_BF16 / AW4_F16 / AW4_F64) and "any" (run
// time).  Specialised kernels take the first three; float64 runs the generic kernels only.
enum : int { D_F32 = AW4_F32, D_BF16 = AW4_BF16, D_F16 = AW4_F16, D_F64 = AW4_F64, D_ANY = 7 };

// Launch table staged in device memory: header, tensors[count], tile_start[count + 1].
struct StepHeader {
    int32_t count;
    int32_t cb1, lut1, cb2, lut2;  // codebook / lookup table of each moment (specialised kernels)
    int32_t reserved;
    int64_t total_tiles;
    int64_t tiles_per_wave;
};

// ---------------------------------------------------------------------------
// 4-value vector access (streaming: each byte is touched once per step)
// ---------------------------------------------------------------------------

// Raw 32-bit words of 4 values: fp32 values, or 2 words of packed 16-bit values.
template <int D>
__device__ __forceinline__ void load_words(uint64_t base, int64_t e, bool vec, uint32_t* w) {
    if constexpr (D == D_F32) {
        const gptr<const float> p = gaddr<const float>(base) + e;
        if (vec) {
            const u32x4 v = __builtin_nontemporal_load((gptr<const u32x4>)p);
            w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) w[t] = f2u(p[t]);
        }
    } else {
        const gptr<const uint16_t> p = gaddr<const uint16_t>(base) + e;
        if (vec) {
            const u32x2 v = __builtin_nontemporal_load((gptr<const u32x2>)p);
            w[0] = v.x; w[1] = v.y;
        } else {
            w[0] = (uint32_t)p[0] | ((uint32_t)p[1] << 16);
            w[1] = (uint32_t)p[2] | ((uint32_t)p[3] << 16);
        }
    }
}

template <int D>
__device__ __forceinline__ void words_to_f32(const uint32_t* w, float (&o)[4]) {
    if constexpr (D == D_F32) {
#pragma unroll
        for (int t = 0; t < 4; ++t) o[t] = u2f(w[t]);
    } else if constexpr (D == D_BF16) {
        o[0] = bf16_to_f32(w[0] & 0xffffu); o[1] = bf16_to_f32(w[0] >> 16);
        o[2] = bf16_to_f32(w[1] & 0xffffu); o[3] = bf16_to_f32(w[1] >> 16);
    } else {
        o[0] = f16_to_f32(w[0] & 0xffffu); o[1] = f16_to_f32(w[0] >> 16);
        o[2] = f16_to_f32(w[1] & 0xffffu); o[3] = f16_to_f32(w[1] >> 16);
    }
}

template <int D>
__device__ __forceinline__ void store_f32(uint64_t base, int64_t e, bool vec, const float (&v)[4]) {
    if constexpr (D == D_F32) {
        const gptr<float> p = gaddr<float>(base) + e;
        if (vec) {
            __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, (gptr<f32x4>)p);
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) p[t] = v[t];
        }
    } else {
        uint32_t h[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) h[t] = D == D_BF16 ? f32_to_bf16(v[t]) : f32_to_f16(v[t]);
        const gptr<uint16_t> p = gaddr<uint16_t>(base) + e;
        if (vec) {
            if constexpr (D == D_BF16)
                __builtin_nontemporal_store(u32x2{f32x2_to_bf16x2(v[0], v[1]), f32x2_to_bf16x2(v[2], v[3])},
                                            (gptr<u32x2>)p);
            else
                __builtin_nontemporal_store(u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)}, (gptr<u32x2>)p);
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) p[t] = (uint16_t)h[t];
        }
    }
}

template <int D>
__device__ __forceinline__ float round_to_storage(float v) {
    if constexpr (D == D_BF16) return bf16_to_f32(f32_to_bf16(v));
    else if constexpr (D == D_F16) return f16_to_f32(f32_to_f16(v));
    else return v;
}

__device__ __forceinline__ float round_to_dtype(float v, int dt) {
    return dt == D_BF16 ? round_to_storage<D_BF16>(v) : dt == D_F16 ? round_to_storage<D_F16>(v) : v;
}

// Loss-scale unscaling and gradient clipping applied as the step reads the gradients
// (grad_scale -> {u, c}): with AW4_TENSOR_GRAD_UNSCALE g -> grad_dtype(fp32(g * u)), the value
// GradScaler.unscale_'s _amp_foreach_non_finite_check_and_unscale_ leaves in a gradient of
// that dtype (u = its fp32 inverse scale); then with AW4_TENSOR_GRAD_SCALE g ->
// grad_dtype(fp32(g * c)), what the in-place _foreach_mul_ of torch.nn.utils.clip_grad_norm_
// leaves (the fp32 product of two 16-bit values is exact, so one rounding to the dtype each).
// G is the gradient's storage dtype, D_ANY for a run-time one.  The branch is uniform per tensor.
template <int G>
__device__ __forceinline__ void clip_grads(const aw4_tensor& T, float* g, int n) {
    if (__builtin_expect((T.flags & (AW4_TENSOR_GRAD_SCALE | AW4_TENSOR_GRAD_UNSCALE)) == 0, 1)) return;
    const gptr<const float> f = gaddr<const float>(T.grad_scale);
    const float u = f[0], c = f[1];
    const bool unscale = (T.flags & AW4_TENSOR_GRAD_UNSCALE) != 0, clip = (T.flags & AW4_TENSOR_GRAD_SCALE) != 0;
    const int dt = G == D_ANY ? T.grad_dtype : G;
    for (int t = 0; t < n; ++t) {
        float v = g[t];
        if (unscale) v = round_to_dtype(v * u, dt);
        if (clip) v = round_to_dtype(v * c, dt);
        g[t] = v;
    }
}

// float64 values: 4 at element e (vec: two 16-byte accesses).
__device__ __forceinline__ void load_f64x4(uint64_t base, int64_t e, bool vec, double (&d)[4]) {
    const gptr<const double> p = gaddr<const double>(base) + e;
    if (vec) {
        const f64x2 a = __builtin_nontemporal_load((gptr<const f64x2>)p);
        const f64x2 b = __builtin_nontemporal_load((gptr<const f64x2>)(p + 2));
        d[0] = a.x; d[1] = a.y; d[2] = b.x; d[3] = b.y;
    } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) d[t] = p[t];
    }
}

__device__ __forceinline__ void store_f64x4(uint64_t base, int64_t e, bool vec, const double (&d)[4]) {
    const gptr<double> p = gaddr<double>(base) + e;
    if (vec) {
        __builtin_nontemporal_store(f64x2{d[0], d[1]}, (gptr<f64x2>)p);
        __builtin_nontemporal_store(f64x2{d[2], d[3]}, (gptr<f64x2>)(p + 2));
    } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) p[t] = d[t];
    }
}

// Run-time dtype dispatch for the generic kernel (D_ANY): loads convert to fp32 words (a
// float64 gradient rounded to nearest, as gradient.to(float32)).  A float64 parameter is not
// loaded here: its update reads it in float64 (update_quarter).
__device__ __forceinline__ void load_words_any(int dtype, uint64_t base, int64_t e, bool vec, uint32_t* w) {
    uint32_t r[4];
    float f[4];
    if (dtype == D_F32) {
        load_words<D_F32>(base, e, vec, w);
        return;
    }
    if (dtype == D_F64) {
        double d[4];
        load_f64x4(base, e, vec, d);
#pragma unroll
        for (int t = 0; t < 4; ++t) w[t] = f2u((float)d[t]);
        return;
    }
    if (dtype == D_BF16) {
        load_words<D_BF16>(base, e, vec, r);
        words_to_f32<D_BF16>(r, f);
    } else {
        load_words<D_F16>(base, e, vec, r);
        words_to_f32<D_F16>(r, f);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) w[t] = f2u(f[t]);
}

// ---------------------------------------------------------------------------
// AdamW arithmetic of one value (_optimized.py:215-222, ATen operation order)
// ---------------------------------------------------------------------------

// m1 = lerp(m1, g, 1-beta1); m2 = lerp(m2, g*g, 1-beta2): ATen's lerp is one fused
// multiply-add, fma(w, end - start, start) for |w| < 0.5 and fma(w - 1, end - start, end)
// otherwise (the host passes w - 1 and sets the LERP*_LARGE flag).
template <bool kLarge1, bool kLarge2>
__device__ __forceinline__ void moments_update(const aw4_tensor& T, float g, float& m1, float& m2) {
    const float gg = g * g;
    m1 = __builtin_fmaf(T.w1, g - m1, kLarge1 ? g : m1);
    m2 = __builtin_fmaf(T.w2, gg - m2, kLarge2 ? gg : m2);
}

// p = p * (1 - lr*wd) [rounded to storage]; p = p + (-lr/bc1 * m1) / (sqrt(m2) / sqrt(bc2) + eps).
// The denominator and the quotient are faithful: hardware square root and reciprocal
// (<= 1 ulp each), so the update term is within 3 ulps of ATen's, whose square root is
// itself only faithful; the sum is one fused operation.  The decayed parameter is exact; the
// update term is usually far below its ulp.  Zero, infinite and NaN denominators give ATen's
// results (x * rcp(0) = x / 0, x * rcp(inf) = 0 for finite x).
__device__ __forceinline__ float param_apply(const aw4_tensor& T, float p1, float m1, float m2) {
    const float d = __builtin_fmaf(sqrt_faithful(m2), T.bc2_sqrt_rcp, T.eps);
    return __builtin_fmaf(T.step_coef * m1, __builtin_amdgcn_rcpf(d), p1);
}

template <int D>
__device__ __forceinline__ float param_update(const aw4_tensor& T, float p, float m1, float m2) {
    return param_apply(T, round_to_storage<D>(p * T.decay), m1, m2);
}

// A float64 parameter (AW4_F64; the reference's eager chunk update, _optimized.py:219-222): the
// fp32 denominator fp32(sqrt(m2)) / fp32(sqrt(bc2)) + fp32(eps) (a true division, as ATen's
// div_ by a Python scalar), then p = p * (1 - lr*wd) and p = p + ((-lr/bc1) * m1) / den with
// m1 and den widened, every operation rounded to float64 (ATen's CPU addcdiv order; hipcc
// contracts nothing and divides float64 correctly rounded).  The root is the correctly rounded
// one, which ATen's CPU root also gives on all but a few percent of inputs (1 ulp below it
// there); v_sqrt_f32 alone is off by an ulp far more often, and a float64 parameter shows it.
__device__ __forceinline__ float denominator_f64_param(const aw4_tensor& T, float m2) {
    return div_cr(sqrt_cr(m2), T.bc2_sqrt) + T.eps;
}

__device__ __forceinline__ double param_update_f64(const aw4_tensor& T, double p, float m1, float den) {
    const double p1 = p * T.decay_f64;
    return p1 + (T.step_coef_f64 * (double)m1) / (double)den;
}

// The decayed parameters p * (1 - lr*wd) of 4 values, rounded to storage (bf16: one conversion
// for two values).
template <int D>
__device__ __forceinline__ void decay4(const aw4_tensor& T, const float (&p)[4], float (&p1)[4]) {
    if constexpr (D == D_BF16 || D == D_F16) {
        // 1 - 2^-9 < decay <= 1 (bf16; 1 - 2^-12 for fp16): p * decay is within half a storage ulp of
        // every 16-bit p (the spacing below a power of two, the closest case, is 2^-8 of it for
        // bf16, 2^-11 for fp16; subnormals have a wider relative spacing), so it rounds back to p.
        // The branch is uniform, and the test compares bit patterns (scalar integer compares:
        // positive floats order as their bits, and a negative or NaN decay fails it).
        constexpr uint32_t kIdentity = D == D_BF16 ? 0x3F7F8000u : 0x3F7FF000u;  // 1 - 2^-9, 1 - 2^-12
        const uint32_t db = f2u(T.decay);
        if (db > kIdentity && db <= 0x3F800000u) {
#pragma unroll
            for (int t = 0; t < 4; ++t) p1[t] = p[t];
            return;
        }
    }
    if constexpr (D == D_BF16) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t w = f32x2_to_bf16x2(p[2 * h] * T.decay, p[2 * h + 1] * T.decay);
            p1[2 * h] = u2f(w << 16);
            p1[2 * h + 1] = u2f(w & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) p1[t] = round_to_storage<D>(p[t] * T.decay);
    }
}

// ---------------------------------------------------------------------------
// Tiles of tensors whose numel is a multiple of 128 (block layout)
// ---------------------------------------------------------------------------

// Whether a kernel moves parts of a tile between memory and its lanes through LDS: the specialised
// bf16 kernels of the recipes (not the read-back or lookahead m2 ones).  Their lanes own 4 values
// of a quarter, 8 bytes, so that direct accesses touch half of each 128-byte line per instruction
// and the code words come in 2-byte loads.  Instead each lane loads one 8-byte piece of the tile's
// codes and stores the 16-byte pieces of updated parameters 64 h + 8 j .. + 7 of its block, and
// codes_to_lanes / params_to_memory rearrange them in LDS.  (Loading the gradients and
// parameters the same way measured no faster, for 6 more registers.)
constexpr bool lds_tile_io(int m1k, int m2k, int d) {
    return d == D_BF16 && kind_of(m1k) != K_ANY && kind_of(m2k) != K_ANY && kind_of(m2k) != K_LA &&
           (flags_of(m2k) & AW4_MOMENT_SAMPLED_READ) == 0;
}
// Whether a kernel loads its code bytes as one 8-byte piece per lane (codes_to_lanes): the
// lds_tile_io kernels, and the fp32 update-SR kernels of the recipes, where it replaces eight
// 2-byte loads per lane and tile (Llama-3-8B ZIP-SR: 20.70 -> 20.38 ms per launch).  The fp32
// round-to-nearest kernels keep the 2-byte loads: the code words' registers made them spill.
constexpr bool lds_code_io(int m1k, int m2k, int d) {
    return lds_tile_io(m1k, m2k, d) ||
           (d == D_F32 && kind_of(m1k) != K_ANY && kind_of(m2k) == K_USR && (flags_of(m2k) & AW4_MOMENT_SAMPLED_READ) == 0);
}

// Raw inputs of one lane for one wave tile (blocks blk0 .. blk0+7; lane's block blk0 + lane/8).
template <int M1K, int M2K, int D>
struct TileInputs {
    static constexpr int kW = (D == D_F32 || D == D_ANY) ? 4 : 2;  // words per 4 values
    static constexpr int K1 = kind_of(M1K), K2 = kind_of(M2K);
    // a pending lookahead m2 (AW4_MOMENT_PENDING in its spec) keeps fp32 values, no codes
    static constexpr bool kQ1 = K1 != K_FP32, kV1 = K1 == K_FP32 || K1 == K_ANY;
    static constexpr bool kQ2 = K2 != K_FP32 && !pending_spec(M2K), kV2 = K2 == K_FP32 || K2 == K_ANY || pending_spec(M2K);
    uint32_t g[4 * kW];
    uint32_t p[4 * kW];
    uint32_t c1[kQ1 ? 2 : 1], c2[kQ2 ? 2 : 1];  // code words of quarters 2h (low half) and 2h + 1 (high half)
    float s1, s2;
    float v1[kV1 ? 16 : 1], v2[kV2 ? 16 : 1];
};

// Whether the moment's state is codes and scales (else fp32 values: an fp32-state moment, or
// a pending lookahead m2).
__device__ __forceinline__ bool is_quantized(const aw4_moment& m) { return has_codes(m.rounding, m.flags); }

template <int MK>
__device__ __forceinline__ bool moment_quantized(const aw4_moment& m) {
    if constexpr (kind_of(MK) == K_ANY) return is_quantized(m);
    else return kind_of(MK) != K_FP32 && !pending_spec(MK);
}

// Addressing of one lane within a wave tile: the tile's base pointers are wave-uniform
// (scalar registers), the lane offsets 32-bit (values: grp*128 + 4j + 32q; code bytes:
// grp*64 + 2j + 16q; scales: grp).
struct TileLane {
    int j, grp;
    bool active;     // the lane's block exists (the last tile of a tensor may be partial)
    int64_t blk0;    // first block of the tile (uniform)
    uint32_t voff;   // value offset of (q = 0, t = 0) from the tile's first value
};

__device__ __forceinline__ TileLane tile_lane(const aw4_tensor& T, int64_t blk0, int lane) {
    TileLane tl;
    tl.j = lane & 7;
    tl.grp = lane >> 3;
    tl.blk0 = blk0;
    tl.active = blk0 + tl.grp < (T.numel >> 7);
    tl.voff = (uint32_t)(tl.grp * kBlock + 4 * tl.j);
    return tl;
}

template <int D>
__device__ __forceinline__ uint64_t tile_values(uint64_t base, int64_t blk0) {
    return base + (uint64_t)blk0 * kBlock * (D == D_F32 ? 4 : 2);
}

template <int M1K, int M2K, int D>
__device__ __forceinline__ void load_tile(const aw4_tensor& T, const TileLane& tl, TileInputs<M1K, M2K, D>& in) {
    using In = TileInputs<M1K, M2K, D>;
    const bool vec = D != D_ANY || (T.flags & AW4_TENSOR_VEC_ALIGNED) != 0;  // specialised kernels: host-checked
    // Lanes past a tensor's last block (only in its last tile) read the tile's first block,
    // which always exists, so every register holds loaded data without a fill or a masked
    // load; their results are never stored, and every block statistic stays within one
    // block's 8 lanes.
    const uint32_t voff = tl.active ? tl.voff : 4u * (uint32_t)tl.j;
    const int grp = tl.active ? tl.grp : 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t off = voff + 32u * q;
        if constexpr (D == D_ANY) {
            const int64_t e = tl.blk0 * kBlock + off;
            load_words_any(T.grad_dtype, T.grad, e, vec, &in.g[4 * q]);
            if (T.param_dtype != D_F64) load_words_any(T.param_dtype, T.param, e, vec, &in.p[4 * q]);
        } else {
            load_words<D>(tile_values<D>(T.grad, tl.blk0), off, true, &in.g[In::kW * q]);
            load_words<D>(tile_values<D>(T.param, tl.blk0), off, true, &in.p[In::kW * q]);
        }
    }
    auto load_moment = [&](const aw4_moment& M, uint32_t* c, float& s, float* v, auto quant, auto vals) {
        constexpr bool kQ = decltype(quant)::value, kV = decltype(vals)::value;
        bool quantized = kQ;
        if constexpr (kQ && kV) quantized = is_quantized(M);
        if (quantized) {
            if constexpr (kQ) {
                const gptr<const uint8_t> codes = gaddr<const uint8_t>(M.codes) + tl.blk0 * (kBlock / 2);
                if constexpr (lds_code_io(M1K, M2K, D)) {
                    // The tile's code bytes in memory order, one 8-byte load per lane (bytes 8 l .. 8 l + 7
                    // of the tile: the words of one quarter for four lanes of block l / 8); codes_to_lanes
                    // hands each lane its own four words through LDS before they are decoded.
                    const u32x2 w = __builtin_nontemporal_load(
                        (gptr<const u32x2>)(codes + 8u * (uint32_t)(grp * kBlocksPerWave + tl.j)));
                    c[0] = w.x;
                    c[1] = w.y;
                } else {
                    const uint32_t coff = (uint32_t)(grp * (kBlock / 2) + 2 * tl.j);
                    // two 16-bit code words per register: 4 fewer registers per tile in flight
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint32_t lo = __builtin_nontemporal_load((gptr<const uint16_t>)(codes + coff + 32u * h));
                        const uint32_t hi =
                            __builtin_nontemporal_load((gptr<const uint16_t>)(codes + coff + 32u * h + 16u));
                        c[h] = lo | (hi << 16);
                    }
                }
                s = (gaddr<const float>(M.scales) + tl.blk0)[grp];
            }
        } else {
            if constexpr (kV) {
                const gptr<const float> vals_tile = gaddr<const float>(M.values) + tl.blk0 * kBlock;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const f32x4 x = __builtin_nontemporal_load((gptr<const f32x4>)(vals_tile + voff + 32u * q));
                    v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
                }
            }
        }
    };
    load_moment(T.m1, in.c1, in.s1, in.v1, std::integral_constant<bool, In::kQ1>(),
                std::integral_constant<bool, In::kV1>());
    load_moment(T.m2, in.c2, in.s2, in.v2, std::integral_constant<bool, In::kQ2>(),
                std::integral_constant<bool, In::kV2>());
}

// Byte offset of 16-byte column c (0..15) of block grp in a tile image of 16-bit values held in
// LDS (256 bytes per block): the column index is XORed with the block so that the 8 blocks' lanes,
// which access the same columns of their blocks, spread over the banks.
__device__ __forceinline__ uint32_t image_column(int grp, int c) { return (uint32_t)(grp * 256 + ((c ^ grp) << 4)); }

// The code words of a loaded tile, from memory order to their lanes (lds_code_io kernels):
// load_tile leaves lane l (block l / 8) with bytes 8 l .. 8 l + 7 of the tile's codes; lane j of
// block grp decodes the words at bytes 64 grp + 16 q + 2 j (q = 0..3), two to a register (quarters
// 2h, 2h + 1).  The bytes go through the wave's scratch, which no encode of this tile uses yet;
// lanes past a tensor's last block (which loaded block 0's bytes) read block 0's words, as every
// other input of theirs.
template <int M1K, int M2K, int D>
__device__ __forceinline__ void codes_to_lanes(const aw4_tensor& T, const TileLane& tl, TileInputs<M1K, M2K, D>& in,
                                               WaveScratch& ws) {
    if constexpr (!lds_code_io(M1K, M2K, D)) return;
    using In = TileInputs<M1K, M2K, D>;
    const bool q1 = In::kQ1 && moment_quantized<M1K>(T.m1), q2 = In::kQ2 && moment_quantized<M2K>(T.m2);
    if (!q1 && !q2) return;
    uint8_t* buf = ws.code_words();
    const int lane = tl.grp * kBlocksPerWave + tl.j;
    wave_lds_sync();  // earlier readers of the scratch are done
    if (q1) *(u32x2*)(buf + 8 * lane) = u32x2{in.c1[0], in.c1[1]};
    if (q2) *(u32x2*)(buf + kWaveCodeBytes + 8 * lane) = u32x2{in.c2[0], in.c2[1]};
    wave_lds_sync();
    const uint32_t base = (uint32_t)((tl.active ? tl.grp : 0) * (kBlock / 2) + 2 * tl.j);
    auto words = [&](const uint8_t* b, uint32_t* c) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t lo = *(const uint16_t*)(b + base + 32u * h);
            const uint32_t hi = *(const uint16_t*)(b + base + 32u * h + 16u);
            c[h] = lo | (hi << 16);
        }
    };
    if constexpr (In::kQ1) {
        if (q1) words(buf, in.c1);
    }
    if constexpr (In::kQ2) {
        if (q2) words(buf + kWaveCodeBytes, in.c2);
    }
    wave_lds_sync();  // the words are read before the scratch is written again
}

// The updated parameters of a tile to memory (lds_tile_io kernels): update_quarter left each
// lane's 8-byte pieces in a parameter image in the wave's scratch (image_column); each lane stores
// the 16-byte pieces of values 64 h + 8 j .. + 7 of its block (the host runs these kernels only
// where the parameter is 16-byte aligned).  Before the tile's encodes use the scratch.
template <int M1K, int M2K, int D>
__device__ __forceinline__ void params_to_memory(const aw4_tensor& T, const TileLane& tl, WaveScratch& ws) {
    if constexpr (!lds_tile_io(M1K, M2K, D)) return;
    const uint8_t* img = ws.code_words();
    wave_lds_sync();
    if (tl.active) {
        const gptr<uint16_t> pt =
            gaddr<uint16_t>(tile_values<D>(T.param, tl.blk0)) + (uint32_t)(tl.grp * kBlock + 8 * tl.j);
#pragma unroll
        for (int h = 0; h < 2; ++h)
            __builtin_nontemporal_store(*(const u32x4*)(img + image_column(tl.grp, 8 * h + tl.j)),
                                        (gptr<u32x4>)(pt + 64u * h));
    }
    wave_lds_sync();  // the pieces are read before the encodes write the scratch
}

template <int MK, bool kNonNeg, class Values>
__device__ __forceinline__ BlockScales encode_moment(const aw4_moment& M, const MomentTables& L, const TileLane& tl,
                                                     const Values& v, BlockScratch sc) {
    if constexpr (kind_of(MK) == K_ANY) return encode_block_any<kNonNeg>(M, L, tl.blk0, tl.grp, tl.j, tl.active, v, sc);
    else return encode_block<MK, kNonNeg>(M, L, tl.blk0, tl.grp, tl.j, tl.active, v, sc);
}

// Where the update puts the new second moments: registers, or this lane's slots of an LDS
// stage (quarter-major, 64 lanes per quarter: conflict-free 16-byte accesses) with their
// running max |v| for the encode.
struct M2Regs {
    float (&m)[16];
    __device__ void put(int q, const float (&b)[4]) {
#pragma unroll
        for (int t = 0; t < 4; ++t) m[4 * q + t] = b[t];
    }
    __device__ RegValues values() const { return RegValues{m}; }
};
struct M2Staged {
    f32x4* lane_q0;
    float amax;
    __device__ void put(int q, const float (&b)[4]) {
        lane_q0[64 * q] = f32x4{b[0], b[1], b[2], b[3]};
#pragma unroll
        for (int t = 0; t < 4; ++t) amax = abs_max_acc(amax, b[t]);
    }
    __device__ StagedValues values() const { return StagedValues{lane_q0, amax}; }
};

// Decode, update and store one quarter (4 values) of this lane; the new moments go to m1/m2.
// kDefer: the parameter update waits for the stored m2 (AW4_MOMENT_SAMPLED_READ); p1 receives
// the decayed parameters and nothing is stored.
// la_prior (pending lookahead m2): the samples of the pending state; the new m2 is then
// fp32(beta2) * sample + fp32(1-beta2) * g * g in ATen's addcmul form
// fma(fp32(1-beta2) * g, g, fp32(beta2) * sample) (adamw.py:576).
template <int M1K, int M2K, int D, int DP, bool kGenericLerp, bool kDefer, class M2Sink>
__device__ __forceinline__ void update_quarter(const aw4_tensor& T, int q, const TileInputs<M1K, M2K, D>& in,
                                               const MomentTables& L1, const MomentTables& L2, const TileLane& tl,
                                               float (&m1)[16], M2Sink& m2, float* p1, const float* la_prior,
                                               uint8_t* p_img) {
    using In = TileInputs<M1K, M2K, D>;
    constexpr int DC = D == D_ANY ? D_F32 : D;  // generic loads are already fp32 words
    constexpr bool kF64 = DP == D_F64;  // the parameter is read, updated and stored in float64 below
    float g[4], p[4], a[4], b[4];
    words_to_f32<DC>(&in.g[In::kW * q], g);
    clip_grads<D>(T, g, 4);
    if constexpr (!kF64) words_to_f32<DC>(&in.p[In::kW * q], p);
    if (moment_quantized<M1K>(T.m1)) {
        if constexpr (In::kQ1) decode4(L1.dec, in.c1[q >> 1] >> (16 * (q & 1)), in.s1, a);
    } else {
        if constexpr (In::kV1) {
#pragma unroll
            for (int t = 0; t < 4; ++t) a[t] = in.v1[4 * q + t];
        }
    }
    if (moment_quantized<M2K>(T.m2)) {
        if constexpr (In::kQ2) decode4(L2.dec, in.c2[q >> 1] >> (16 * (q & 1)), in.s2, b);
    } else {
        if constexpr (In::kV2) {
#pragma unroll
            for (int t = 0; t < 4; ++t) b[t] = in.v2[4 * q + t];
        }
    }
    const bool large1 = (T.flags & AW4_TENSOR_LERP1_LARGE) != 0, large2 = (T.flags & AW4_TENSOR_LERP2_LARGE) != 0;
    float pd[4];
    if constexpr (!kF64) decay4<DP>(T, p, pd);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        if constexpr (kGenericLerp) {
            const float gg = g[t] * g[t];
            a[t] = __builtin_fmaf(T.w1, g[t] - a[t], large1 ? g[t] : a[t]);
            b[t] = __builtin_fmaf(T.w2, gg - b[t], large2 ? gg : b[t]);
        } else {
            moments_update<false, false>(T, g[t], a[t], b[t]);
        }
        if (la_prior)
            b[t] = __builtin_fmaf((float)T.m2.la_fresh_weight * g[t], g[t], la_prior[4 * q + t] * (float)T.m2.la_beta2);
        if constexpr (kF64) {
            if constexpr (!kDefer) p[t] = denominator_f64_param(T, b[t]);  // the update follows the store of m2
        } else if constexpr (kDefer) {
            p1[4 * q + t] = pd[t];
        } else {
            p[t] = param_apply(T, pd[t], a[t], b[t]);
        }
        m1[4 * q + t] = a[t];
    }
    m2.put(q, b);
    if (!kDefer && tl.active) {
        const uint32_t off = tl.voff + 32u * q;
        if constexpr (kF64) {
            // (the generic kernel: D_ANY) p holds the denominators
            const bool vec = (T.flags & AW4_TENSOR_VEC_ALIGNED) != 0;
            const int64_t e = tl.blk0 * kBlock + off;
            double v[4];
            load_f64x4(T.param, e, vec, v);
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = param_update_f64(T, v[t], a[t], p[t]);
            store_f64x4(T.param, e, vec, v);
        } else if constexpr (D == D_ANY) {
            const bool vec = (T.flags & AW4_TENSOR_VEC_ALIGNED) != 0;
            const int64_t e = tl.blk0 * kBlock + off;
            if (T.param_dtype == D_F32) store_f32<D_F32>(T.param, e, vec, p);
            else if (T.param_dtype == D_BF16) store_f32<D_BF16>(T.param, e, vec, p);
            else store_f32<D_F16>(T.param, e, vec, p);
        } else if constexpr (lds_tile_io(M1K, M2K, D)) {
            // the 8-byte piece into the tile's parameter image (params_to_memory stores it)
            *(u32x2*)(p_img + image_column(tl.grp, 4 * q + (tl.j >> 1)) + 8u * (uint32_t)(tl.j & 1)) =
                u32x2{f32x2_to_bf16x2(p[0], p[1]), f32x2_to_bf16x2(p[2], p[3])};
        } else {
            store_f32<D>(tile_values<D>(T.param, tl.blk0), off, true, p);
        }
    }
}

template <int M1K, int M2K, int D, int DP, bool kDefer, class M2Sink>
__device__ __forceinline__ void update_tile(const aw4_tensor& T, const TileInputs<M1K, M2K, D>& in,
                                            const MomentTables& L1, const MomentTables& L2, const TileLane& tl,
                                            float (&m1)[16], M2Sink& m2, float* p1, const float* la_prior,
                                            uint8_t* p_img) {
    if (__builtin_expect((T.flags & (AW4_TENSOR_LERP1_LARGE | AW4_TENSOR_LERP2_LARGE)) == 0, 1)) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            update_quarter<M1K, M2K, D, DP, false, kDefer>(T, q, in, L1, L2, tl, m1, m2, p1, la_prior, p_img);
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            update_quarter<M1K, M2K, D, DP, true, kDefer>(T, q, in, L1, L2, tl, m1, m2, p1, la_prior, p_img);
    }
}

// Decode, update and store the parameters of one tile; the new moments go to m1/m2.
template <int M1K, int M2K, int D, bool kDefer = false, class M2Sink>
__device__ __forceinline__ void update_tile_any(const aw4_tensor& T, const TileLane& tl,
                                                const TileInputs<M1K, M2K, D>& in, const MomentTables& L1,
                                                const MomentTables& L2, float (&m1)[16], M2Sink& m2,
                                                float* p1 = nullptr, const float* la_prior = nullptr,
                                                uint8_t* p_img = nullptr) {
    if constexpr (D == D_ANY) {
        if (T.param_dtype == D_F32) update_tile<M1K, M2K, D, D_F32, kDefer>(T, in, L1, L2, tl, m1, m2, p1, la_prior, p_img);
        else if (T.param_dtype == D_BF16)
            update_tile<M1K, M2K, D, D_BF16, kDefer>(T, in, L1, L2, tl, m1, m2, p1, la_prior, p_img);
        else if (T.param_dtype == D_F16)
            update_tile<M1K, M2K, D, D_F16, kDefer>(T, in, L1, L2, tl, m1, m2, p1, la_prior, p_img);
        else update_tile<M1K, M2K, D, D_F64, kDefer>(T, in, L1, L2, tl, m1, m2, p1, la_prior, p_img);
    } else {
        update_tile<M1K, M2K, D, D, kDefer>(T, in, L1, L2, tl, m1, m2, p1, la_prior, p_img);
    }
}

// The gradients of this lane's 16 values as fp32.
template <int M1K, int M2K, int D>
__device__ __forceinline__ void tile_grads(const aw4_tensor& T, const TileInputs<M1K, M2K, D>& in, float (&g)[16]) {
    using In = TileInputs<M1K, M2K, D>;
    constexpr int DC = D == D_ANY ? D_F32 : D;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float v[4];
        words_to_f32<DC>(&in.g[In::kW * q], v);
        clip_grads<D>(T, v, 4);
#pragma unroll
        for (int t = 0; t < 4; ++t) g[4 * q + t] = v[t];
    }
}

// Parameter update of a tile whose m2 is read back after its encode (AW4_MOMENT_SAMPLED_READ,
// adamw.py:636-656): v = cb[code] * scale from the code words the encode left in the
// block's LDS stage (scale: the stored one, or with AW4_MOMENT_READ_RAW_SCALE the one before
// EDEN, adamw.py:615-635), d = sqrt(v) / sqrt(bc2) + eps, p = p1 + (step_coef * m1) / d
// (correctly rounded divisions, as the reference's), and 1 / d to M.values when it is set
// (m2_read_preconditioner, adamw.py:632).  A float64 parameter (DP = D_F64; p1 is not used) is
// read here and updated in float64 (param_update_f64).
template <int DP>
__device__ __forceinline__ void sampled_read_update(const aw4_tensor& T, const TileLane& tl, const MomentTables& L2,
                                                    BlockScratch sc, BlockScales bs, const float (&m1)[16],
                                                    const float (&p1)[16]) {
    const float stored = __shfl(bs.stored, (int)(threadIdx.x & 63) & ~7);  // lane j == 0 of the block
    const float scale = (T.m2.flags & AW4_MOMENT_READ_RAW_SCALE) ? bs.raw : stored;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float v[4], p[4], den[4];
        decode4(L2.dec, sc.stage[8 * q + tl.j], scale, v);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float sq = DP == D_F64 ? sqrt_cr(v[t]) : sqrt_faithful(v[t]);  // see denominator_f64_param
            const float d = __builtin_amdgcn_div_fixupf(div_by_rcp(sq, T.bc2_sqrt, T.bc2_sqrt_rcp), T.bc2_sqrt, sq) + T.eps;
            if constexpr (DP != D_F64) p[t] = p1[4 * q + t] + div_cr(T.step_coef * m1[4 * q + t], d);
            den[t] = d;
        }
        if (tl.active) {
            const uint32_t off = tl.voff + 32u * q;
            const bool vec = (T.flags & AW4_TENSOR_VEC_ALIGNED) != 0;
            if constexpr (DP == D_F64) {
                double w[4];
                load_f64x4(T.param, tl.blk0 * kBlock + off, vec, w);
#pragma unroll
                for (int t = 0; t < 4; ++t) w[t] = param_update_f64(T, w[t], m1[4 * q + t], den[t]);
                store_f64x4(T.param, tl.blk0 * kBlock + off, vec, w);
            } else {
                store_f32<DP>(T.param, tl.blk0 * kBlock + off, vec, p);
            }
            if (T.m2.values) {  // only the read-back schemes that keep 1 / denominator
                float pre[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) pre[t] = div_cr(1.0f, den[t]);
                *(gptr<f32x4>)(gaddr<float>(T.m2.values) + tl.blk0 * kBlock + off) = f32x4{pre[0], pre[1], pre[2], pre[3]};
            }
        }
    }
}

// Encode (or store, for an fp32-state moment) one moment of a tile.
template <int MK, bool kNonNeg, class Values>
__device__ __forceinline__ BlockScales finish_moment(const aw4_moment& M, const MomentTables& L, const TileLane& tl,
                                                     const Values& v, WaveScratch& ws) {
    if (moment_quantized<MK>(M)) {
        if constexpr (kind_of(MK) != K_FP32) return encode_moment<MK, kNonNeg>(M, L, tl, v, ws.block(tl.grp));
    } else if (tl.active) {
        const gptr<float> vals_tile = gaddr<float>(M.values) + tl.blk0 * kBlock;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float x[4];
            v.quarter(q, x);
            __builtin_nontemporal_store(f32x4{x[0], x[1], x[2], x[3]}, (gptr<f32x4>)(vals_tile + tl.voff + 32u * q));
        }
    }
    return BlockScales{0.0f, 0.0f};
}

// ---------------------------------------------------------------------------
// Tiles of fp32-state tensors with any numel (values e_tile .. e_tile + 1023)
// ---------------------------------------------------------------------------

template <int D>
__device__ __forceinline__ float load_value(const aw4_tensor& T, uint64_t base, int dtype, int64_t k) {
    const int dt = D == D_ANY ? dtype : D;
    if (dt == D_F32) return gaddr<const float>(base)[k];
    if (D == D_ANY && dt == D_F64) return (float)gaddr<const double>(base)[k];
    const uint32_t h = gaddr<const uint16_t>(base)[k];
    return dt == D_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

template <int D>
__device__ __forceinline__ void step_values_one(const aw4_tensor& T, int64_t k) {
    const gptr<float> v1 = gaddr<float>(T.m1.values);
    const gptr<float> v2 = gaddr<float>(T.m2.values);
    float g = load_value<D>(T, T.grad, T.grad_dtype, k);
    clip_grads<D>(T, &g, 1);
    const int dt = D == D_ANY ? T.param_dtype : D;
    float p = dt == D_F64 ? 0.0f : load_value<D>(T, T.param, T.param_dtype, k);
    float a = v1[k], b = v2[k];
    const int lf = T.flags & (AW4_TENSOR_LERP1_LARGE | AW4_TENSOR_LERP2_LARGE);
    if (lf == 0) moments_update<false, false>(T, g, a, b);
    else if (lf == AW4_TENSOR_LERP1_LARGE) moments_update<true, false>(T, g, a, b);
    else if (lf == AW4_TENSOR_LERP2_LARGE) moments_update<false, true>(T, g, a, b);
    else moments_update<true, true>(T, g, a, b);
    if (D == D_ANY && dt == D_F64) {
        const gptr<double> pp = gaddr<double>(T.param);
        pp[k] = param_update_f64(T, pp[k], a, denominator_f64_param(T, b));
    } else if (dt == D_F32) {
        p = param_update<D_F32>(T, p, a, b);
        gaddr<float>(T.param)[k] = p;
    } else if (dt == D_BF16) {
        p = param_update<D_BF16>(T, p, a, b);
        gaddr<uint16_t>(T.param)[k] = (uint16_t)f32_to_bf16(p);
    } else {
        p = param_update<D_F16>(T, p, a, b);
        gaddr<uint16_t>(T.param)[k] = (uint16_t)f32_to_f16(p);
    }
    v1[k] = a;
    v2[k] = b;
}

// Out of line (a cold path); the row is read through a global pointer, so that its fields are
// global loads here too (a generic one would give flat instructions).
template <int D>
__device__ void step_tile_values(gptr<const aw4_tensor> row, int64_t e_tile, int lane) {
    const aw4_tensor& T = *(const aw4_tensor*)row;
    const int j = lane & 7;
    const int grp = lane >> 3;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t e = e_tile + grp * kBlock + 32 * q + 4 * j;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            if (e + t < T.numel) step_values_one<D>(T, e + t);
    }
}

// ---------------------------------------------------------------------------
// The kernel: wave w of a grid of W waves processes tiles w, w + W, w + 2W, ... (at most
// the header's tiles_per_wave; the grid covers every tile).  The waves resident at any
// moment have consecutive indices, so the tiles in flight are adjacent in memory, while
// each workgroup's table load is shared by several tiles per wave.  Latency is hidden by
// occupancy (several waves per SIMD) and by issuing the next tile's loads as soon as the
// current tile's inputs are dead (after the parameter update and the first moment's
// encode): the second moment's encode then overlaps them, and its code and scale stores
// queue behind them, so waiting for those loads does not wait for these stores (on gfx9
// one counter covers both, in issue order).
// ---------------------------------------------------------------------------

// Tiles of tensors without block structure: both moments fp32 state, or numel not a
// multiple of 128.  (Written through has_codes: the equivalent comparisons with K_FP32
// lead hipcc to copy the prefetched tile registers instead of coalescing them, 40 more
// VGPRs in the specialised kernels; the resource test pins the counts.)
__device__ __forceinline__ bool values_only(const aw4_tensor& T) {
    return (!has_codes(T.m1.rounding, 0) && !has_codes(T.m2.rounding, 0)) || (T.numel & (kBlock - 1)) != 0;
}

// Tile order: grid order (wave w takes tiles w, w + W, ...) or consecutive tiles per wave
// (w * K .. w * K + K - 1).  Prefetch: the next tile's loads are issued during the second
// moment's encode.  Both keep the in-flight tiles of a memory-bound kernel adjacent and
// its loads early.  The bf16 update-SR kernels, bound by their instruction issue, take
// consecutive tiles (grid order cost them 2% at twelve tiles per wave, for its per-tile tensor
// search).  The generic kernel (run-time kinds and dtype) has the register pressure of every
// variant at once and loads each tile when it starts it.
// Kernel instances for the reference step's research m2 variants: m2 read back after its
// encode (AW4_MOMENT_SAMPLED_READ in the m2 spec's flags) and lookahead update-SR
// (AW4_ROUND_LOOKAHEAD_SR); the generic one (any kind, marked by the flag) runs both.
constexpr bool research_kernel(int m2k) {
    return (flags_of(m2k) & AW4_MOMENT_SAMPLED_READ) != 0 || kind_of(m2k) == K_LA;
}
// (Not for the research m2 variants: the registers of a prefetched tile leave the read-back
// kernels at 2 waves per SIMD, 21% slower than 3 without the prefetch.)
constexpr bool prefetch_next_tile(int m1k, int m2k, int d) {
    return kind_of(m1k) != K_ANY && kind_of(m2k) != K_ANY && d != D_ANY && !research_kernel(m2k);
}
constexpr bool tile_order_grid(int m1k, int m2k, int d) {
    return prefetch_next_tile(m1k, m2k, d) && !(kind_of(m2k) == K_USR && d == D_BF16);
}
// Update-SR kernels stage the new second moments in LDS (M2Staged) so that the prefetched
// inputs fit in the registers of four waves per SIMD.
constexpr bool stage_m2(int m1k, int m2k, int d) { return prefetch_next_tile(m1k, m2k, d) && kind_of(m2k) == K_USR; }

// Index of the tensor holding `tile` >= tile_start[lo]: the last ti in [lo, count) with
// tile_start[ti] <= tile (one load when it is still tensor lo, else a binary search).
__device__ __forceinline__ int tensor_of(const int64_t* tile_start, int lo, int count, int64_t tile) {
    if (tile < tile_start[lo + 1]) return lo;
    ++lo;
    int hi = count - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tile_start[mid] <= tile) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// `load_tables` fills the workgroup's LDS tables and synchronises the workgroup: every wave
// calls it exactly once, after issuing its first tile's loads, so those loads are in flight
// during the table load.
template <int M1K, int M2K, int D, class LdsT, class LoadTables>
__device__ __forceinline__ void run_tiles(const StepHeader* hdr, const LdsT& lds_tables, WaveScratch& ws,
                                          f32x4* m2_stage, LoadTables&& load_tables) {
    const aw4_tensor* tensors = (const aw4_tensor*)(hdr + 1);
    const int count = hdr->count;
    const int64_t* tile_start = (const int64_t*)(tensors + count);
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * kWavesPerGroup + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Tile order and prefetch of this variant (tile_order_grid, prefetch_next_tile).
    constexpr bool kGridOrder = tile_order_grid(M1K, M2K, D), kPrefetch = prefetch_next_tile(M1K, M2K, D);
    const int64_t stride = kGridOrder ? (int64_t)gridDim.x * kWavesPerGroup : 1;
    const int64_t total = hdr->total_tiles;
    const int64_t per_wave = hdr->tiles_per_wave;
    int64_t tile = kGridOrder ? wave : wave * per_wave;
    const bool any = tile < total;
    int ti = any ? tensor_of(tile_start, 0, count, tile) : 0;
    TileInputs<M1K, M2K, D> in;
    bool loaded = false;  // `in` holds this tile's inputs (issued earlier)
    if (any && !values_only(tensors[ti])) {
        const aw4_tensor& T = tensors[ti];
        load_tile(T, tile_lane(T, (tile - tile_start[ti]) * kBlocksPerWave, lane), in);
        loaded = true;
    }
    load_tables();
    if (!any) return;
    for (int64_t k = 0;;) {
        const aw4_tensor& T = tensors[ti];
        const int64_t local = tile - tile_start[ti];
        const int64_t next = tile + stride;
        const bool more = ++k < per_wave && next < total;
        int tn = -1;  // tensor of `next`, once searched
        if (values_only(T)) {
            step_tile_values<D>((gptr<const aw4_tensor>)&T, local * kWaveTile, lane);
            loaded = false;
        } else {
            const TileLane tl = tile_lane(T, local * kBlocksPerWave, lane);
            if (!loaded) load_tile(T, tl, in);
            codes_to_lanes(T, tl, in, ws);
            const MomentTables L1 = lds_tables.moment(T.m1, 0);
            const MomentTables L2 = lds_tables.moment(T.m2, 1);
            auto prefetch = [&]() {
                loaded = false;
                if (kPrefetch && more) {
                    tn = tensor_of(tile_start, ti, count, next);
                    const aw4_tensor& Tn = tensors[tn];
                    if (!values_only(Tn)) {
                        load_tile(Tn, tile_lane(Tn, (next - tile_start[tn]) * kBlocksPerWave, lane), in);
                        loaded = true;
                    }
                }
            };
            float m1[16];
            if constexpr (research_kernel(M2K)) {
                // every block tile of this kernel has a research m2 (the host groups them)
                float m2v[16];
                M2Regs m2{m2v};
                bool sampled = false;  // m2 read back after its encode (else lookahead)
                if constexpr (kind_of(M2K) != K_LA) sampled = (T.m2.flags & AW4_MOMENT_SAMPLED_READ) != 0;
                if constexpr (kind_of(M2K) != K_LA) {
                  if (sampled) {
                    float p1[16];
                    update_tile_any<M1K, M2K, D, true>(T, tl, in, L1, L2, m1, m2, p1);
                    finish_moment<M1K, false>(T.m1, L1, tl, RegValues{m1}, ws);
                    prefetch();
                    const BlockScales bs = finish_moment<M2K, true>(T.m2, L2, tl, m2.values(), ws);
                    const int dp = D == D_ANY ? T.param_dtype : D;  // a specialised kernel's own dtype
                    if (dp == D_F32) sampled_read_update<D_F32>(T, tl, L2, ws.block(tl.grp), bs, m1, p1);
                    else if (dp == D_BF16) sampled_read_update<D_BF16>(T, tl, L2, ws.block(tl.grp), bs, m1, p1);
                    else if (dp == D_F16) sampled_read_update<D_F16>(T, tl, L2, ws.block(tl.grp), bs, m1, p1);
                    else if (D == D_ANY) sampled_read_update<D_F64>(T, tl, L2, ws.block(tl.grp), bs, m1, p1);
                  }
                }
                if constexpr (kind_of(M2K) == K_ANY || kind_of(M2K) == K_LA) {
                  if (!sampled) {
                    // lookahead update-SR: sample the pending state before the update (the
                    // generic instance, or the K_LA instance specialised on AW4_MOMENT_PENDING),
                    // or encode the new m2 after it (the code-storing proxies)
                    constexpr bool kMaybePending = kind_of(M2K) == K_ANY || pending_spec(M2K);
                    float g[16];
                    tile_grads(T, in, g);
                    const bool pending = pending_spec(M2K) ||
                                         (kind_of(M2K) == K_ANY && (T.m2.flags & AW4_MOMENT_PENDING) != 0);
                    const float w2f = (float)T.m2.la_fresh_weight;
                    float prior[16];
                    if constexpr (kMaybePending) {
                        if (pending) {
                            float z[16];
#pragma unroll
                            for (int i = 0; i < 16; ++i) z[i] = in.v2[i];
                            encode_block_la(T.m2, L2, tl.blk0, tl.grp, tl.j, tl.active, z, g, w2f, false, prior,
                                            ws.block(tl.grp));
                        }
                    }
                    update_tile_any<M1K, M2K, D, false>(T, tl, in, L1, L2, m1, m2, nullptr, pending ? prior : nullptr);
                    finish_moment<M1K, false>(T.m1, L1, tl, RegValues{m1}, ws);
                    prefetch();
                    bool stored = false;
                    if constexpr (kMaybePending) {
                        if (pending) {
                            finish_moment<M2K, true>(T.m2, L2, tl, m2.values(), ws);
                            stored = true;
                        }
                    }
                    if constexpr (!pending_spec(M2K)) {
                        if (!stored)
                            encode_block_la(T.m2, L2, tl.blk0, tl.grp, tl.j, tl.active, m2v, g, w2f, true, nullptr,
                                            ws.block(tl.grp));
                    }
                  }
                }
            } else if constexpr (stage_m2(M1K, M2K, D)) {
                M2Staged m2{m2_stage + lane, 0.0f};
                update_tile_any(T, tl, in, L1, L2, m1, m2, nullptr, nullptr, ws.code_words());
                params_to_memory<M1K, M2K, D>(T, tl, ws);
                finish_moment<M1K, false>(T.m1, L1, tl, RegValues{m1}, ws);
                prefetch();
                finish_moment<M2K, true>(T.m2, L2, tl, m2.values(), ws);
            } else {
                float m2v[16];
                M2Regs m2{m2v};
                update_tile_any(T, tl, in, L1, L2, m1, m2, nullptr, nullptr, ws.code_words());
                params_to_memory<M1K, M2K, D>(T, tl, ws);
                finish_moment<M1K, false>(T.m1, L1, tl, RegValues{m1}, ws);
                prefetch();
                finish_moment<M2K, true>(T.m2, L2, tl, m2.values(), ws);
            }
        }
        if (!more) break;
        ti = tn >= 0 ? tn : tensor_of(tile_start, ti, count, next);
        tile = next;
    }
}

}  // namespace aw4
