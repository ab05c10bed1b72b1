// Fused 4-bit AdamW step for MI355X (gfx950): one multi-tensor launch per optimizer step.
//
// Work decomposition
//   * A 128-value block (one fp32 scale per moment) is owned by 8 lanes of a 64-lane
//     wave; a wave owns 8 consecutive blocks (a 1024-value wave tile).
//   * Lane j (0..7) of a block owns the 16 values at offsets 32q + 4j + t (q, t = 0..3):
//     every parameter/gradient access is a 4-value vector (16 B for fp32) and each
//     quarter q of a block is one contiguous 128 B segment across the 8 lanes.  The same
//     split makes the reference's per-block sum order (ATen's 8-lane x 4-accumulator
//     reduction) mostly lane-local (block_sum_cross in aw4_math.h).
//   * Tiles of all tensors form one index space; each wave takes up to 4 tiles (in grid
//     order for the memory-bound kernels, consecutive ones for the update-SR kernels) and
//     the grid covers all of them, so the hardware dispatcher keeps the tiles in flight a
//     narrow moving window of memory.  One launch covers every parameter of the step,
//     fp32-state tensors included.
//   * Kernels are specialised on (m1 rounding kind, m2 rounding kind, parameter dtype);
//     a launch table whose tensors share one such combination (every recipe) runs the
//     specialised kernel, any other table the generic one.
//
// Arithmetic contract (the reference's ATen CPU operations, in order):
//   decode    m = cb[code] * scale                       (_optimized_quantization.py:91-107)
//   moments   m1 = fma(w1, g - m1, m1); m2 = fma(w2, g*g - m2, m2)   (ATen lerp)
//   denom     d = sqrt(m2) / sqrt(bc2) + eps             (_optimized.py:219-220)
//   param     p = p * (1 - lr*wd); p = p + (step_coef * m1) / d      (_optimized.py:221-222)
//   encode    s = max(max|m|, 1e-12); x = m / s; round; [dyn4_nz floor]; [EDEN]
//             (_optimized_quantization.py:46-88, _compiled_quantization.py:30-109)
// The file is compiled with -ffp-contract=off: every fused multiply-add is explicit.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <string>
#include <algorithm>
#include <type_traits>
#include <vector>

#include "adamw4bit_hip.h"
#ifndef AW4_SCHED_ILP_TU
#include "aw4_prologue.h"  // its kernels belong to the main object only
#endif
#include "aw4_step.h"

// Device memory the library holds without allocating it: file-scope arrays, one copy per GPU,
// kept until the process ends.  g_tables_mem holds the codebook and lookup tables every kernel
// reads; `scratch` holds the launch tables of aw4_fused_step_noalloc.  In host code these names
// are stand-ins, not device addresses: the host takes each GPU's address of them with
// hipGetSymbolAddress (device_state) and uses only that.  (Only the main object holds them: the
// second compile of this file, AW4_SCHED_ILP_TU below, emits kernels and nothing else.)
#ifndef AW4_SCHED_ILP_TU
static __device__ __align__(256) uint8_t g_tables_mem[sizeof(aw4::Tables)];
static __device__ __align__(256) uint8_t scratch[AW4_NOALLOC_TABLE_BYTES];
#endif

namespace {

using namespace aw4;

static_assert(sizeof(aw4_moment) == 104, "aw4_moment layout");
static_assert(sizeof(aw4_tensor) == 296, "aw4_tensor layout");

// Codebooks as fp32 bit patterns (ascending; code = index).  Values of the reference's
// closed forms: NF4 table (quantization.py:401-422), signed and unsigned dynamic maps
// with 3 exponent bits (:201-237), linspace grids (:457-497).
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

// Lookup table a moment encodes with: round-to-nearest (dyn4_nz: floored) or level count.
__host__ __device__ inline int lut_id_of(int rounding, int codebook, int flags) {
    if (rounding == AW4_ROUND_RTN)
        return ((flags & AW4_MOMENT_ZERO_FLOOR) && codebook == AW4_CB_DYN4) ? kLutRtnDyn4Floor : kLutRtn[codebook];
    return kLutLevels[codebook];
}

// ---------------------------------------------------------------------------
// LDS layouts
// ---------------------------------------------------------------------------

// Specialised kernels: the tables of the one codebook each moment uses.
template <bool kUpd>
struct LdsSlots {
    float cb[2][16];
    UsrPair usr[2][kPairs];
    PairEntry pairs[2][kPairs];
    float2 dec[2][256];
    LutEntry lut[2][AW4_LUT_ENTRIES];
    WaveScratch scratch[kWavesPerGroup];
    f32x4 m2_stage[kUpd ? kWavesPerGroup * 4 * 64 : 1];  // second moments of a tile (update-SR kernels)

    __device__ MomentTables moment(const aw4_moment&, int which) const {
        return MomentTables{cb[which], pairs[which], dec[which], lut[which], usr[which]};
    }
    __device__ f32x4* wave_m2_stage(int wslot) { return kUpd ? &m2_stage[wslot * 4 * 64] : nullptr; }
    __device__ void load(const Tables* g, const StepHeader* h) {
        const int cbs[2] = {h->cb1, h->cb2}, luts[2] = {h->lut1, h->lut2};
        for (int w = 0; w < 2; ++w) {
            if (cbs[w] < 0) continue;
            for (int i = threadIdx.x; i < 16; i += kThreads) cb[w][i] = g->codebook[cbs[w]][i];
            for (int i = threadIdx.x; i < kPairs; i += kThreads) usr[w][i] = g->usr[cbs[w]][i];
            for (int i = threadIdx.x; i < kPairs; i += kThreads) pairs[w][i] = g->pairs[cbs[w]][i];
            for (int i = threadIdx.x; i < 256; i += kThreads) dec[w][i] = g->dec[cbs[w]][i];
            for (int i = threadIdx.x; i < AW4_LUT_ENTRIES; i += kThreads) lut[w][i] = g->lut[luts[w]][i];
        }
        __syncthreads();
    }
};

// Generic kernels: every table.
struct LdsAll {
    Tables t;
    WaveScratch scratch[kWavesPerGroup];

    __device__ __forceinline__ MomentTables moment(const aw4_moment& m, int) const {
        const int cbid = m.rounding == AW4_ROUND_FP32 ? 0 : m.codebook;
        return MomentTables{t.codebook[cbid], t.pairs[cbid], t.dec[cbid],
                            t.lut[m.rounding == AW4_ROUND_FP32 ? 0 : lut_id_of(m.rounding, cbid, m.flags)],
                            t.usr[cbid]};
    }
    __device__ f32x4* wave_m2_stage(int) { return nullptr; }
    __device__ void load(const Tables* g, const StepHeader*) {
        const uint32_t* src = (const uint32_t*)g;
        uint32_t* dst = (uint32_t*)&t;
        for (int i = threadIdx.x; i < (int)(sizeof(Tables) / 4); i += kThreads) dst[i] = src[i];
        __syncthreads();
    }
};

template <int M1K, int M2K, int D>
struct KernelTraits {
    static constexpr int K1 = kind_of(M1K), K2 = kind_of(M2K);
    static constexpr bool kGeneric = K1 == K_ANY || K2 == K_ANY || D == D_ANY;
    static constexpr bool kUpd = K1 == K_USR || K2 == K_USR || K1 == K_ANY || K2 == K_ANY;
    using Lds = typename std::conditional<kGeneric, LdsAll, LdsSlots<kUpd>>::type;
};

template <int M1K, int M2K, int D>
__device__ __forceinline__ void step_body(const StepHeader* __restrict__ hdr, const Tables* __restrict__ tables) {
    using Lds = typename KernelTraits<M1K, M2K, D>::Lds;
    __shared__ Lds lds;
    const int wslot = threadIdx.x >> 6;
    run_tiles<M1K, M2K, D>(hdr, lds, lds.scratch[wslot], lds.wave_m2_stage(wslot), [&] { lds.load(tables, hdr); });
}

template <int M1K, int M2K, int D>
__global__ void __launch_bounds__(kThreads) step_kernel(const StepHeader* __restrict__ hdr,
                                                         const Tables* __restrict__ tables) {
    step_body<M1K, M2K, D>(hdr, tables);
}

// The same kernel held to 128 VGPRs, four waves per SIMD (the fp32 recipes fit without spills;
// the fourth wave hides memory latency the third leaves exposed).
template <int M1K, int M2K, int D>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4)))
step_kernel_4w(const StepHeader* __restrict__ hdr, const Tables* __restrict__ tables) {
    step_body<M1K, M2K, D>(hdr, tables);
}

// The same kernel held to 256 VGPRs, two waves per SIMD: the generic research instance (every
// m2 kind, read back or lookahead, with run-time dtypes) needs 270 otherwise, one wave per SIMD;
// the few registers it spills cost less than the second wave gains (pending lookahead 108 ->
// 66 ms on the Llama-3-8B set).
template <int M1K, int M2K, int D>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
step_kernel_2w(const StepHeader* __restrict__ hdr, const Tables* __restrict__ tables) {
    step_body<M1K, M2K, D>(hdr, tables);
}

// The same kernel held to 168 VGPRs, three waves per SIMD: the pending lookahead instance needs
// 178 otherwise (two waves); six registers spill, and the third wave takes its step on the
// Llama-3-8B set from 37.8 to 34.8 ms.
template <int M1K, int M2K, int D>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3)))
step_kernel_3w(const StepHeader* __restrict__ hdr, const Tables* __restrict__ tables) {
    step_body<M1K, M2K, D>(hdr, tables);
}

// Small steps: the launch table travels in the kernel arguments, so that the step is one launch
// with no staging copy before it and no staging buffer to recycle after it (the launch packet
// holds its own copy of the arguments).  The kernel reads the table where the arguments are, so
// its fields still come through scalar loads.  Instances exist for the two recipes' kernels.
constexpr int kInlineTableBytes = 3584;

struct __align__(16) InlineArgs {
    const Tables* tables;
    uint64_t reserved;
    unsigned char table[kInlineTableBytes];
};

template <int M1K, int M2K, int D>
__device__ __forceinline__ void step_body_inline(const InlineArgs& a) {
    const StepHeader* hdr =
        (const StepHeader*)((const char*)__builtin_amdgcn_kernarg_segment_ptr() + offsetof(InlineArgs, table));
    step_body<M1K, M2K, D>(hdr, a.tables);
}

template <int M1K, int M2K, int D>
__global__ void __launch_bounds__(kThreads) step_kernel_inline(const InlineArgs a) {
    step_body_inline<M1K, M2K, D>(a);
}

template <int M1K, int M2K, int D>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4)))
step_kernel_inline_4w(const InlineArgs a) {
    step_body_inline<M1K, M2K, D>(a);
}

}  // namespace

// The four-wave update-SR kernels (ZIP-SR's fp32 and bf16 steps, the bf16 nf4_sr head and
// EDEN-m2 ablation) come from a second compile of this file, with AW4_SCHED_ILP_TU defined and
// LLVM's max-ilp machine scheduler (-mllvm -amdgpu-sched-strategy=max-ilp); that object holds
// nothing else.  Bound by their instruction issue, they ran 1.2-1.5% faster under it (ZIP-SR on
// the Llama-3-8B fp32 set 19.40-19.55 against 19.77-19.85 ms, the bf16 set 16.28-16.49 against
// 16.49-16.72 ms per step; alternating processes on one box, five each), while ZE-EDEN spills
// under it and ran 4% slower, so every other kernel keeps the default scheduler.  The main
// object declares them and launches them through the variant table.
namespace aw4_ilp {
template <int M1K, int M2K, int D>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4)))
step_kernel_4w(const aw4::StepHeader* __restrict__ hdr, const aw4::Tables* __restrict__ tables)
#ifdef AW4_SCHED_ILP_TU
{
    step_body<M1K, M2K, D>(hdr, tables);
}
#else
    ;
#endif
}  // namespace aw4_ilp

namespace {

// The instantiated kernels; the host groups a step's tensors by the variant whose moment
// specs and dtype they match (optimized-path flags).  ZE-EDEN: NF4 round-to-nearest m1,
// Dyn4 round-to-nearest m2 with EDEN.  ZIP-SR: NF4 round-to-nearest m1, Dyn4 update-SR m2
// with the exact-level guards; its nf4_sr head (value-space SR m1).  QuantizedAdamW
// ablations of ZIP-SR: an fp32 m2, EDEN on the update-SR m2.
constexpr int kRtn = mspec(K_RTN), kRtnEden = mspec(K_RTN, AW4_MOMENT_EDEN), kFp32 = mspec(K_FP32);
constexpr int kSsrGuarded = mspec(K_SSR, AW4_MOMENT_GUARDS);
constexpr int kUsrGuarded = mspec(K_USR, AW4_MOMENT_GUARDS);
constexpr int kUsrGuardedEden = mspec(K_USR, AW4_MOMENT_GUARDS | AW4_MOMENT_EDEN);
// The reference step's update-SR m2 read back after its encode: dyn4_upd_sr / lin4_upd_sr,
// and *_upd_sr_store_eden (read at the scale before EDEN, EDEN on the stored scale).
constexpr int kUsrRead = mspec(K_USR, AW4_MOMENT_SAMPLED_READ);
constexpr int kUsrReadEden = mspec(K_USR, AW4_MOMENT_SAMPLED_READ | AW4_MOMENT_READ_RAW_SCALE | AW4_MOMENT_EDEN);
// Lookahead update-SR m2 stored as codes (dyn4_proxy_la_upd_sr, dyn4_vproxy_la_upd_sr).
constexpr int kLaStore = mspec(K_LA);
// ... and the pending form (dyn4_la_upd_sr): fp32 state sampled before the update.
constexpr int kLaPending = mspec(K_LA, AW4_MOMENT_PENDING);
// Any m2 kind of the research schemes (read-back and lookahead), any dtype.
constexpr int kAnyResearch = mspec(K_ANY, AW4_MOMENT_SAMPLED_READ);

#ifdef AW4_SCHED_ILP_TU
}  // namespace

template __global__ void aw4_ilp::step_kernel_4w<kRtn, kUsrGuarded, D_F32>(const aw4::StepHeader*, const aw4::Tables*);
template __global__ void aw4_ilp::step_kernel_4w<kRtn, kUsrGuarded, D_BF16>(const aw4::StepHeader*, const aw4::Tables*);
template __global__ void aw4_ilp::step_kernel_4w<kSsrGuarded, kUsrGuarded, D_BF16>(const aw4::StepHeader*,
                                                                                   const aw4::Tables*);
template __global__ void aw4_ilp::step_kernel_4w<kRtn, kUsrGuardedEden, D_BF16>(const aw4::StepHeader*,
                                                                                const aw4::Tables*);
#else

struct KernelVariant {
    int m1, m2, dtype;
    const void* fn;
    const void* fn_inline;  // the instance taking its table in the arguments, or null
};
#define AW4_VARIANT(M1, M2, D) {M1, M2, D, (const void*)&step_kernel<M1, M2, D>, nullptr}
#define AW4_VARIANT_4W(M1, M2, D) {M1, M2, D, (const void*)&step_kernel_4w<M1, M2, D>, nullptr}
#define AW4_VARIANT_2W(M1, M2, D) {M1, M2, D, (const void*)&step_kernel_2w<M1, M2, D>, nullptr}
#define AW4_VARIANT_3W(M1, M2, D) {M1, M2, D, (const void*)&step_kernel_3w<M1, M2, D>, nullptr}
#define AW4_VARIANT_I(M1, M2, D) \
    {M1, M2, D, (const void*)&step_kernel<M1, M2, D>, (const void*)&step_kernel_inline<M1, M2, D>}
#define AW4_VARIANT_I4W(M1, M2, D) \
    {M1, M2, D, (const void*)&step_kernel_4w<M1, M2, D>, (const void*)&step_kernel_inline_4w<M1, M2, D>}
// the max-ilp instances of the second object (their small-step instances stay in this one)
#define AW4_VARIANT_ILP(M1, M2, D) {M1, M2, D, (const void*)&aw4_ilp::step_kernel_4w<M1, M2, D>, nullptr}
#define AW4_VARIANT_ILP_I4W(M1, M2, D) \
    {M1, M2, D, (const void*)&aw4_ilp::step_kernel_4w<M1, M2, D>, (const void*)&step_kernel_inline_4w<M1, M2, D>}
const KernelVariant kVariants[] = {
    AW4_VARIANT_I4W(kRtn, kRtnEden, D_F32),       AW4_VARIANT_ILP_I4W(kRtn, kUsrGuarded, D_F32),
    AW4_VARIANT_I4W(kRtn, kRtnEden, D_BF16),      AW4_VARIANT_ILP_I4W(kRtn, kUsrGuarded, D_BF16),
    AW4_VARIANT(kSsrGuarded, kUsrGuarded, D_F32), AW4_VARIANT_ILP(kSsrGuarded, kUsrGuarded, D_BF16),
    AW4_VARIANT(kRtn, kFp32, D_F32),              AW4_VARIANT(kRtn, kFp32, D_BF16),
    AW4_VARIANT(kRtn, kUsrGuardedEden, D_F32),    AW4_VARIANT_ILP(kRtn, kUsrGuardedEden, D_BF16),
    AW4_VARIANT(kRtn, kUsrRead, D_F32),           AW4_VARIANT(kRtn, kUsrReadEden, D_F32),
    AW4_VARIANT(kRtn, kLaStore, D_F32),           AW4_VARIANT_3W(kRtn, kLaPending, D_F32),
    AW4_VARIANT_2W(K_ANY, kAnyResearch, D_ANY),
    AW4_VARIANT(K_ANY, K_ANY, D_ANY),
};
#undef AW4_VARIANT
#undef AW4_VARIANT_4W
#undef AW4_VARIANT_2W
#undef AW4_VARIANT_3W
#undef AW4_VARIANT_I
#undef AW4_VARIANT_I4W
#undef AW4_VARIANT_ILP
#undef AW4_VARIANT_ILP_I4W
constexpr int kNumVariants = sizeof(kVariants) / sizeof(kVariants[0]);
constexpr int kGenericVariant = kNumVariants - 1;
constexpr int kResearchVariant = kNumVariants - 2;  // generic, for read-back and lookahead m2
constexpr int kNumSpecialised = kResearchVariant;

// Stand-alone codec kernels (one wave tile per wave, grid-stride).
__global__ void __launch_bounds__(kThreads) quantize_kernel(const float* __restrict__ values, int64_t numel,
                                                            aw4_moment M, const Tables* __restrict__ tables) {
    __shared__ LdsAll lds;
    lds.load(tables, nullptr);
    const int lane = threadIdx.x & 63;
    const int wslot = threadIdx.x >> 6;
    const int j = lane & 7, grp = lane >> 3;
    const int64_t nblocks = numel / kBlock;
    const int64_t tiles = (nblocks + kBlocksPerWave - 1) / kBlocksPerWave;
    const int64_t nwaves = (int64_t)gridDim.x * kWavesPerGroup;
    const MomentTables L = lds.moment(M, 0);
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
        // stand-alone encodes accept any sign (a first moment or a caller's values)
        encode_block_any<false>(M, L, tile * kBlocksPerWave, grp, j, active, RegValues{m}, lds.scratch[wslot].block(grp));
    }
}

__global__ void __launch_bounds__(kThreads) dequantize_kernel(aw4_moment M, int64_t numel, float* __restrict__ out,
                                                              const Tables* __restrict__ tables) {
    __shared__ LdsAll lds;
    lds.load(tables, nullptr);
    const int lane = threadIdx.x & 63;
    const int wslot = threadIdx.x >> 6;
    const int j = lane & 7, grp = lane >> 3;
    const int64_t nblocks = numel / kBlock;
    const int64_t tiles = (nblocks + kBlocksPerWave - 1) / kBlocksPerWave;
    const int64_t nwaves = (int64_t)gridDim.x * kWavesPerGroup;
    const MomentTables L = lds.moment(M, 0);
    for (int64_t tile = (int64_t)blockIdx.x * kWavesPerGroup + wslot; tile < tiles; tile += nwaves) {
        const int64_t blk = tile * kBlocksPerWave + grp;
        if (blk >= nblocks) continue;
        uint32_t w[4];
        const gptr<const uint8_t> codes = gaddr<const uint8_t>(M.codes) + blk * (kBlock / 2) + 2 * j;
#pragma unroll
        for (int q = 0; q < 4; ++q) w[q] = *(gptr<const uint16_t>)(codes + 16 * q);
        const float scale = gaddr<const float>(M.scales)[blk];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float m[4];
            decode4(L.dec, w[q], scale, m);
            *(float4*)(out + blk * kBlock + 32 * q + 4 * j) = make_float4(m[0], m[1], m[2], m[3]);
        }
    }
}

// Uniforms at positions offset .. offset+n-1 (n > 0): one thread per (position group, lane).
__global__ void __launch_bounds__(kThreads) uniforms_kernel(uint64_t seed, uint64_t offset, int64_t n,
                                                            float* __restrict__ out) {
    const uint64_t g0 = offset >> 7, end = offset + (uint64_t)n;
    const int64_t lanes = (int64_t)(((end - 1) >> 7) - g0 + 1) * 8;
    for (int64_t l = (int64_t)blockIdx.x * kThreads + threadIdx.x; l < lanes; l += (int64_t)gridDim.x * kThreads) {
        const uint64_t group = g0 + (uint64_t)(l >> 3);
        const int j = (int)(l & 7);
        uint32_t w[12];
#pragma unroll
        for (int r = 0; r < 3; ++r) philox_lane_call(seed, group, j, r, &w[4 * r]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float u[4];
            lane_fields4(&w[3 * q], u);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint64_t pos = group * kBlock + (uint64_t)(32 * q + 4 * j + t);
                if (pos >= offset && pos < end) out[pos - offset] = u[t] * 0x1p-24f;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

thread_local std::string g_error;
thread_local int g_fail_after = -1;  // aw4_inject_launch_failure

int set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

#define AW4_HIP_CHECK(expr)                                                                             \
    do {                                                                                                \
        hipError_t err_ = (expr);                                                                       \
        if (err_ != hipSuccess) return set_error(AW4_EHIP, "%s: %s", #expr, hipGetErrorString(err_)); \
    } while (0)

float host_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

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
// for every fp32 x of the bucket, where f is monotone non-decreasing in x.  Fails if a
// bucket holds more than one change of f.  The entry's levels are cb[min(f, 15)] for both
// outcomes: the code's level (round-to-nearest) or the upper neighbour b of x (level count).
template <class F>
bool build_lut(LutEntry* out, F f, const float* cb, std::string& err) {
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
            LutEntry e;
            e.base = (uint32_t)base;
            if (top == base) {
                // NaN: x >= thr is false for every x (an infinite threshold would still
                // increment at x = +inf, one past the bucket's count)
                e.thr = host_f(0x7fc00000u);
            } else if (top == base + 1) {
                // smallest x (in value order) with f(x) == base + 1
                uint32_t good = amax, bad = amin;
                while ((sign ? bad - good : good - bad) > 1u) {
                    const uint32_t mid = sign ? good + (bad - good) / 2u : bad + (good - bad) / 2u;
                    if (f(val(mid)) == base + 1) good = mid; else bad = mid;
                }
                e.thr = val(good);
            } else {
                char buf[160];
                snprintf(buf, sizeof(buf), "lookup bucket %d (sign %d) spans %d code changes", k, sign, top - base);
                err = buf;
                return false;
            }
            e.lv_lo = cb[base < 15 ? base : 15];
            e.lv_hi = cb[base + 1 < 15 ? base + 1 : 15];
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
            // square roots of the levels and of their gaps, in double, rounded once to fp32
            float sqrt_level[16];
            for (int k = 0; k < 16; ++k) {
                const double l = (double)t.codebook[c][k];
                sqrt_level[k] = l > 0.0 ? (float)sqrt(l) : 0.0f;
            }
            for (int i = 0; i < kPairs; ++i) {
                const int lo = i > 0 ? i - 1 : 0, hi = i < 15 ? i : 15;
                const double a = (double)t.codebook[c][lo], b = (double)t.codebook[c][hi];
                const float gap = (a >= 0.0 && b > a) ? (float)(sqrt(b) - sqrt(a)) : 0.0f;
                t.usr[c][i] = UsrPair{sqrt_level[lo], sqrt_level[hi], ldexpf(gap, -24),
                                      t.codebook[c][hi] > t.codebook[c][lo] ? 1.0f : 0.0f};
                PairEntry& p = t.pairs[c][i];
                p.a = t.codebook[c][lo];
                p.b = t.codebook[c][hi];
                const float w = p.b - p.a;
                p.width_rcp = 1.0f / (w < 1e-12f ? 1e-12f : w);
                p.lohi = (uint32_t)lo | ((uint32_t)hi << 8);
            }
            for (int b = 0; b < 256; ++b) t.dec[c][b] = make_float2(t.codebook[c][b & 15], t.codebook[c][b >> 4]);
        }
        bool ok = true;
        for (int c = 0; c < AW4_NUM_CODEBOOKS && ok; ++c) {
            const float* cb = t.codebook[c];
            ok = build_lut(t.lut[kLutRtn[c]], [cb](float x) { return rtn_code(cb, x, false); }, cb, h.error) &&
                 build_lut(t.lut[kLutLevels[c]], [cb](float x) { return count_less(cb, x); }, cb, h.error);
        }
        if (ok) {
            const float* cb = t.codebook[AW4_CB_DYN4];
            ok = build_lut(t.lut[kLutRtnDyn4Floor], [cb](float x) { return rtn_code(cb, x, true); }, cb, h.error);
        }
        h.ok = ok;
    });
    return h;
}

struct StagingSlot {
    void* host = nullptr;            // pinned, mapped and coherent: the host writes the table here
    const void* host_dev = nullptr;  // the device's address of `host`
    void* dev = nullptr;             // device copy the kernels read
    size_t cap = 0;
    hipEvent_t done = nullptr;
    bool pending = false;
};

constexpr int kSlots = 4;

struct DeviceState {
    Tables* tables = nullptr;    // this GPU's address of g_tables_mem
    uint8_t* scratch = nullptr;  // this GPU's address of `scratch`
    int num_cus = 0;
    StagingSlot slots[kSlots];
    int next = 0;
    // Host buffers of slots that have grown.  The device has read them uncached; they are kept
    // until the process ends rather than freed and their pages handed out again.
    std::vector<void*> retired_host;
    std::vector<uint8_t> noalloc_host;  // host image of the tables aw4_fused_step_noalloc stages
    std::vector<uint8_t> inline_host;   // host image of the tables of small steps (launch arguments)
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
        // Once per device, with that device current: its addresses of the file-scope arrays, and
        // the codebook tables copied into them (one synchronous copy; nothing is allocated).
        hipDeviceProp_t prop;
        AW4_HIP_CHECK(hipGetDeviceProperties(&prop, dev));
        ds.num_cus = prop.multiProcessorCount;
        void* tables = nullptr;
        void* stage = nullptr;
        AW4_HIP_CHECK(hipGetSymbolAddress(&tables, HIP_SYMBOL(g_tables_mem)));
        AW4_HIP_CHECK(hipGetSymbolAddress(&stage, HIP_SYMBOL(scratch)));
        AW4_HIP_CHECK(hipMemcpy(tables, &ht.t, sizeof(Tables), hipMemcpyHostToDevice));
        ds.scratch = (uint8_t*)stage;
        ds.tables = (Tables*)tables;
    }
    *out = &ds;
    return AW4_OK;
}

bool aligned(uint64_t addr, uint64_t a) { return (addr % a) == 0; }

int check_moment(const aw4_moment& m, int64_t numel, int index, const char* name) {
    const bool la = m.rounding == AW4_ROUND_LOOKAHEAD_SR;
    if ((m.flags & (AW4_MOMENT_FRESH_PROXY | AW4_MOMENT_PENDING)) && !la)
        return set_error(AW4_EINVAL, "tensor %d: %s lookahead flags without lookahead rounding", index, name);
    if (m.rounding == AW4_ROUND_FP32) {
        if (!m.values) return set_error(AW4_EINVAL, "tensor %d: %s fp32 state without values", index, name);
        if (!aligned(m.values, 16)) return set_error(AW4_EALIGN, "tensor %d: %s values not 16-byte aligned", index, name);
        return AW4_OK;
    }
    if (m.rounding < AW4_ROUND_RTN || m.rounding > AW4_ROUND_LOOKAHEAD_SR)
        return set_error(AW4_EINVAL, "tensor %d: %s has rounding %d", index, name, m.rounding);
    if (m.codebook < 0 || m.codebook >= AW4_NUM_CODEBOOKS)
        return set_error(AW4_EINVAL, "tensor %d: %s has codebook %d", index, name, m.codebook);
    if (numel % kBlock != 0)
        return set_error(AW4_EINVAL, "tensor %d: %s quantized but numel %lld is not a multiple of %d", index, name,
                         (long long)numel, kBlock);
    if (la) {
        // lookahead update-SR (quantize_dyn4_la_upd_sr): m2 on the dyn4 codebook only
        if (strcmp(name, "m2") != 0 || m.codebook != AW4_CB_DYN4)
            return set_error(AW4_EINVAL, "tensor %d: lookahead update-SR is for a dyn4 m2 only", index);
        if ((m.flags & AW4_MOMENT_FRESH_PROXY) && (m.flags & AW4_MOMENT_PENDING))
            return set_error(AW4_EINVAL, "tensor %d: m2 FRESH_PROXY and PENDING together", index);
        if (m.flags & (AW4_MOMENT_SAMPLED_READ | AW4_MOMENT_READ_RAW_SCALE | AW4_MOMENT_EDEN))
            return set_error(AW4_EINVAL, "tensor %d: lookahead m2 with read-back or EDEN flags", index);
        if (!(m.la_bias > 0.0) || !(m.la_beta2 >= 0.0 && m.la_beta2 < 1.0) || !(m.la_eps >= 0.0))
            return set_error(AW4_EINVAL, "tensor %d: lookahead m2 needs bias > 0, beta2 in [0, 1), eps >= 0", index);
    }
    if (la && (m.flags & AW4_MOMENT_PENDING)) {
        if (!m.values || !aligned(m.values, 16))
            return set_error(AW4_EINVAL, "tensor %d: pending lookahead m2 without 16-byte aligned values", index);
    } else {
        if (!m.codes || !m.scales)
            return set_error(AW4_EINVAL, "tensor %d: %s quantized without codes/scales", index, name);
        // codes: each lane stores its 16 codes as one 8-byte word
        if (!aligned(m.codes, 8) || !aligned(m.scales, 4))
            return set_error(AW4_EALIGN, "tensor %d: %s codes not 8-byte or scales not 4-byte aligned", index, name);
    }
    if (m.rounding != AW4_ROUND_RTN) {
        if (m.flags & AW4_MOMENT_EXT_DRAWS) {
            if (!m.draws || !aligned(m.draws, 16))
                return set_error(AW4_EINVAL, "tensor %d: %s external draws missing or misaligned", index, name);
        } else if (m.rng_offset % kBlock != 0) {
            return set_error(AW4_EINVAL, "tensor %d: %s rng_offset not a multiple of 128", index, name);
        }
    }
    if (m.rounding == AW4_ROUND_UPDATE_SR && !(m.sr_bias > 0.0f))
        return set_error(AW4_EINVAL, "tensor %d: %s update-SR bias must be positive", index, name);
    if (m.flags & (AW4_MOMENT_SAMPLED_READ | AW4_MOMENT_READ_RAW_SCALE)) {
        if (strcmp(name, "m2") != 0)
            return set_error(AW4_EINVAL, "tensor %d: only m2 can be read back after its encode", index);
        if (!(m.flags & AW4_MOMENT_SAMPLED_READ))
            return set_error(AW4_EINVAL, "tensor %d: m2 READ_RAW_SCALE without SAMPLED_READ", index);
        if (m.values && !aligned(m.values, 16))
            return set_error(AW4_EALIGN, "tensor %d: m2 preconditioner output not 16-byte aligned", index);
    }
    return AW4_OK;
}

int check_tensor(const aw4_tensor& t, int index) {
    if (!t.param || !t.grad) return set_error(AW4_EINVAL, "tensor %d: null param or grad", index);
    if (t.numel <= 0) return set_error(AW4_EINVAL, "tensor %d: numel %lld", index, (long long)t.numel);
    for (int dt : {t.param_dtype, t.grad_dtype})
        if (dt != AW4_F32 && dt != AW4_BF16 && dt != AW4_F16 && dt != AW4_F64)
            return set_error(AW4_EINVAL, "tensor %d: dtype %d", index, dt);
    if (t.flags & AW4_TENSOR_VEC_ALIGNED) {
        // 4-value vector access: 16 bytes (fp32, and float64 as two 16-byte halves) or 8 bytes
        const uint64_t pa = t.param_dtype == AW4_F32 || t.param_dtype == AW4_F64 ? 16 : 8;
        const uint64_t ga = t.grad_dtype == AW4_F32 || t.grad_dtype == AW4_F64 ? 16 : 8;
        if (!aligned(t.param, pa) || !aligned(t.grad, ga))
            return set_error(AW4_EALIGN, "tensor %d: VEC_ALIGNED but param/grad misaligned", index);
    }
    const bool scaled = (t.flags & (AW4_TENSOR_GRAD_SCALE | AW4_TENSOR_GRAD_UNSCALE)) != 0;
    if (scaled && (!t.grad_scale || !aligned(t.grad_scale, 4)))
        return set_error(AW4_EINVAL, "tensor %d: GRAD_SCALE/GRAD_UNSCALE without a 4-byte aligned grad_scale", index);
    if (scaled && t.grad_dtype == AW4_F64)
        return set_error(AW4_EINVAL, "tensor %d: GRAD_SCALE/GRAD_UNSCALE with a float64 gradient", index);
    int rc = check_moment(t.m1, t.numel, index, "m1");
    if (rc) return rc;
    return check_moment(t.m2, t.numel, index, "m2");
}

bool host_values_only(const aw4_tensor& t) {
    return (t.m1.rounding == AW4_ROUND_FP32 && t.m2.rounding == AW4_ROUND_FP32) || t.numel % kBlock != 0;
}

// m2 of the reference step's research variants, stepped by the research kernel instance.
bool research_m2(const aw4_moment& m) {
    return (m.flags & AW4_MOMENT_SAMPLED_READ) || m.rounding == AW4_ROUND_LOOKAHEAD_SR;
}

// One launch of a step: a kernel variant, the tables its LDS slots load, and its tensors.
struct LaunchGroup {
    int variant = kGenericVariant;
    int cb1 = -1, lut1 = -1, cb2 = -1, lut2 = -1;
    std::vector<int> members;
};

// Split a step's tensors into launches: tensors that share a specialised kernel and its
// tables form one launch each; fp32-state tensors join a specialised launch of their
// dtype; everything else (other scheme mixes, fp16, mixed dtypes) runs in one launch of
// the generic kernel.  A recipe's table is one launch.
std::vector<LaunchGroup> plan_launches(const aw4_tensor* ts, int32_t count) {
    std::vector<LaunchGroup> groups;
    LaunchGroup generic, research;
    generic.variant = kGenericVariant;
    research.variant = kResearchVariant;
    std::vector<int> values;
    for (int i = 0; i < count; ++i) {
        const aw4_tensor& t = ts[i];
        if (host_values_only(t)) {
            if (t.param_dtype != t.grad_dtype) generic.members.push_back(i); else values.push_back(i);
            continue;
        }
        const bool research_tensor = research_m2(t.m2);
        const int s1 = mspec(t.m1.rounding, t.m1.flags & spec_flags_mask(t.m1.rounding));
        const int s2 = mspec(t.m2.rounding, t.m2.flags & spec_flags_mask(t.m2.rounding));
        // Specialised kernels access parameters and gradients as 4-value vectors, and those that
        // store parameters through LDS as 16-byte pieces; a row whose addresses do not allow that
        // (a view at an odd offset into a flat buffer) runs the generic kernel, which reads the
        // flag at run time.
        int v = kGenericVariant;
        const bool vec16 = aligned(t.param, 16);
        if (t.param_dtype == t.grad_dtype && (t.flags & AW4_TENSOR_VEC_ALIGNED))
            for (int k = 0; k < kNumSpecialised; ++k)
                if (kVariants[k].dtype == t.param_dtype && kVariants[k].m1 == s1 && kVariants[k].m2 == s2 &&
                    (vec16 || !lds_tile_io(kVariants[k].m1, kVariants[k].m2, kVariants[k].dtype))) {
                    v = k;
                    break;
                }
        if (v == kGenericVariant) { (research_tensor ? research : generic).members.push_back(i); continue; }
        const bool f1 = t.m1.rounding == AW4_ROUND_FP32, f2 = t.m2.rounding == AW4_ROUND_FP32;
        const int c1 = f1 ? -1 : t.m1.codebook, c2 = f2 ? -1 : t.m2.codebook;
        const int l1 = f1 ? -1 : lut_id_of(t.m1.rounding, c1, t.m1.flags);
        const int l2 = f2 ? -1 : lut_id_of(t.m2.rounding, c2, t.m2.flags);
        LaunchGroup* g = nullptr;
        for (LaunchGroup& c : groups)
            if (c.variant == v && c.cb1 == c1 && c.lut1 == l1 && c.cb2 == c2 && c.lut2 == l2) { g = &c; break; }
        if (!g) {
            groups.emplace_back();
            g = &groups.back();
            g->variant = v; g->cb1 = c1; g->lut1 = l1; g->cb2 = c2; g->lut2 = l2;
        }
        g->members.push_back(i);
    }
    for (int i : values) {
        LaunchGroup* g = nullptr;
        for (LaunchGroup& c : groups)
            if (kVariants[c.variant].dtype == ts[i].param_dtype) { g = &c; break; }
        if (!g && !generic.members.empty()) g = &generic;
        if (!g) {
            for (int k = 0; k < kNumSpecialised && !g; ++k) {
                if (kVariants[k].dtype != ts[i].param_dtype) continue;
                groups.emplace_back();
                g = &groups.back();
                g->variant = k;
            }
        }
        (g ? g : &generic)->members.push_back(i);
    }
    if (!research.members.empty()) groups.push_back(std::move(research));
    if (!generic.members.empty()) groups.push_back(std::move(generic));
    for (LaunchGroup& g : groups) std::sort(g.members.begin(), g.members.end());
    return groups;
}

// The next staging slot with at least `bytes` of pinned host and device memory, once the
// launch that last used it has completed.
// Upload of a staged table: a copy kernel on the launch stream reads the pinned host buffer
// directly.  A DMA copy (hipMemcpyAsync) runs on another engine, and the hand-over to it and
// back cost about 20 us each way between consecutive steps (GPT-2-small: 45 us of idle GPU
// per 330 us step, measured).  `cap` is a power of two >= 4096, so the copy's round-up to
// 16 bytes stays inside both buffers.
constexpr int kStageThreads = 256;

__global__ void __launch_bounds__(kStageThreads) stage_copy_kernel(const uint4* src, uint4* dst, int64_t n16) {
    for (int64_t i = (int64_t)blockIdx.x * kStageThreads + threadIdx.x; i < n16;
         i += (int64_t)gridDim.x * kStageThreads)
        dst[i] = src[i];
}

int upload_slot(const StagingSlot& slot, size_t bytes, hipStream_t s) {
    const int64_t n16 = (int64_t)((bytes + 15) / 16);
    if (n16 <= 0) return AW4_OK;
    if ((size_t)n16 * 16 > slot.cap) return set_error(AW4_EINVAL, "staging: %zu bytes exceed the slot", bytes);
    const int64_t blocks = std::min<int64_t>((n16 + kStageThreads - 1) / kStageThreads, 1024);
    hipLaunchKernelGGL(stage_copy_kernel, dim3((unsigned)blocks), dim3(kStageThreads), 0, s,
                       (const uint4*)slot.host_dev, (uint4*)slot.dev, n16);
    AW4_HIP_CHECK(hipGetLastError());
    return AW4_OK;
}

int acquire_slot(DeviceState* ds, size_t bytes, StagingSlot** out) {
    StagingSlot& slot = ds->slots[ds->next];
    ds->next = (ds->next + 1) % kSlots;
    if (slot.pending) {
        AW4_HIP_CHECK(hipEventSynchronize(slot.done));
        slot.pending = false;
    }
    if (slot.cap < bytes) {
        if (slot.host) ds->retired_host.push_back(slot.host);
        if (slot.dev) AW4_HIP_CHECK(hipFree(slot.dev));
        slot.host = slot.dev = nullptr;
        slot.host_dev = nullptr;
        slot.cap = 0;
        size_t cap = 4096;
        while (cap < bytes) cap *= 2;
        // Coherent: the device reads it uncached, so a slot reused four launches later is never
        // read from a stale cache line.
        AW4_HIP_CHECK(hipHostMalloc(&slot.host, cap, hipHostMallocMapped | hipHostMallocCoherent));
        void* mapped = nullptr;
        AW4_HIP_CHECK(hipHostGetDevicePointer(&mapped, slot.host, 0));
        slot.host_dev = mapped;
        AW4_HIP_CHECK(hipMalloc(&slot.dev, cap));
        slot.cap = cap;
    }
    // The event only tells the host that the launch which read the slot has finished; no data
    // flows from the device to the host through it, so it records without a system-scope fence
    // (a cache write-back between consecutive launches).
    if (!slot.done)
        AW4_HIP_CHECK(hipEventCreateWithFlags(&slot.done, hipEventDisableTiming | hipEventDisableSystemFence));
    *out = &slot;
    return AW4_OK;
}

// One step's launches: the kernel groups and where each group's table sits in the staged bytes.
struct StepLaunch {
    std::vector<LaunchGroup> plan;
    std::vector<size_t> offset;
    std::vector<int64_t> grid;
    size_t bytes = 0;
};

// Validate the rows and plan the launches (no device work, no lock needed).
int prepare_step(const aw4_tensor* tensors, int32_t count, StepLaunch& sl) {
    if (count < 0 || (count > 0 && !tensors)) return set_error(AW4_EINVAL, "aw4_fused_step: bad tensor list");
    if (count == 0) return AW4_OK;
    for (int i = 0; i < count; ++i) {
        const int rc = check_tensor(tensors[i], i);
        if (rc) return rc;
    }
    sl.plan = plan_launches(tensors, count);
    // Launch table of each group, 256-byte aligned: header, tensors[n], tile_start[n + 1].
    sl.offset.resize(sl.plan.size());
    sl.grid.assign(sl.plan.size(), 0);
    sl.bytes = 0;
    for (size_t g = 0; g < sl.plan.size(); ++g) {
        const size_t n = sl.plan[g].members.size();
        sl.offset[g] = sl.bytes;
        sl.bytes += (sizeof(StepHeader) + sizeof(aw4_tensor) * n + sizeof(int64_t) * (n + 1) + 255) & ~(size_t)255;
    }
    return AW4_OK;
}

// Tiles per wave of a large launch (per_cu: tiles per CU, at least 128): three for the kernels
// that take their tiles in grid order (all specialised ones but the bf16 update-SR and research
// kernels; bound by memory, or memory and issue together); up to twelve for the
// bf16 update-SR kernels and the research m2 kernels, which are bound by their instruction issue
// and gain from loading each workgroup's tables for more tiles, while a launch keeps at least 128
// tiles per CU for each tile of a wave (several rounds of workgroups, so the last round is a
// small share); four for the rest.  Measured on the Llama-3-8B sets with alternating processes,
// ranked as the first process on a fresh box (where the fp32 set streams slower; two boxes per
// variant), which is how the benchmark runs:
//   ZIP-SR fp32: grid order 2 tiles 21.80-22.09 ms, 3 20.83-21.01, 4 21.10-21.16, 12 21.89-21.90;
//     consecutive tiles 2 21.47, 3 21.16-21.19, 4 21.25-21.37, 8 21.90, 12 21.99-22.00 (in later
//     processes on a box grid order at 4-24 tiles ran 19.1-19.6 ms, consecutive 4 19.7-19.8);
//   ZE-EDEN: grid order 2 20.24-20.44, 3 20.33-20.52, 4 20.49-20.50, 12 as 3 in later processes;
//     consecutive 4 21.14-21.16;
//   the bf16 mixed set (consecutive tiles, later processes): 2 tiles 17.87 ms, 4 16.98-17.07,
//     6 16.80-16.83, 8 16.44-16.65, 12 16.35-16.37, 16 16.28-16.38; in grid order at 12, 2% slower;
//   the research kernels (first process), four -> twelve tiles: proxy lookahead 28.4-28.5 ->
//     27.2-27.4 ms, v-proxy 28.0-28.3 -> 27.4-27.5, pending lookahead 33.5-33.6 -> 32.6-32.7,
//     read-back 23.5-23.7 -> 22.6, store-EDEN 28.0 -> 26.4.
int large_tiles_per_wave(int variant, int64_t per_cu) {
    if (variant < kNumSpecialised) {
        const KernelVariant& kv = kVariants[variant];
        if (tile_order_grid(kv.m1, kv.m2, kv.dtype)) return 3;
        if ((kind_of(kv.m2) == K_USR && kv.dtype == AW4_BF16) || research_kernel(kv.m2))
            return (int)std::max<int64_t>(kTilesPerWave, std::min<int64_t>(12, per_cu / 128));
    }
    return kTilesPerWave;
}

// Write each group's launch table into `dst` (host memory of sl.bytes) and set its grid.
//
// A few tiles per wave and a grid covering all of them: the hardware dispatcher hands each free
// slot the next workgroup, so the tiles in flight stay a narrow, moving window of the index
// space (HBM page locality) and no CU waits on a static share at the end.  Measured on MI355X
// against persistent grids of contiguous per-wave ranges, which stream from thousands of
// far-apart addresses at once and leave a load-imbalance tail.  The kernel picks which tiles a
// wave takes (consecutive ones, or one per grid-sized stride); either way the grid is
// ceil(tiles / tiles per wave) waves.
int fill_step_tables(const aw4_tensor* tensors, StepLaunch& sl, int num_cus, void* dst) {
    for (size_t g = 0; g < sl.plan.size(); ++g) {
        const LaunchGroup& lg = sl.plan[g];
        const int n = (int)lg.members.size();
        StepHeader* h = (StepHeader*)((char*)dst + sl.offset[g]);
        memset(h, 0, sizeof(*h));
        aw4_tensor* rows = (aw4_tensor*)(h + 1);
        int64_t* starts = (int64_t*)(rows + n);
        int64_t acc = 0;
        for (int k = 0; k < n; ++k) {
            rows[k] = tensors[lg.members[k]];
            starts[k] = acc;
            acc += (rows[k].numel + kWaveTile - 1) / kWaveTile;
        }
        starts[n] = acc;
        // Smaller launches take fewer tiles per wave so that their waves still spread over every
        // CU: from 128 tiles per CU 3 or 4; below, one per 16 tiles per CU (16 waves per CU, the
        // four 256-thread workgroups the recipe kernels keep resident: one round of waves), at
        // least 1.  Measured on one 4096^2 ZIP-SR tensor (64 tiles per CU): 4 tiles per wave
        // 52.1-52.2 us, 2 52.7-52.9, 3 56.4-56.6, 1 57.1-57.3; one 1024^2 tensor (4 per CU): 1.
        const int64_t per_cu = acc / (int64_t)num_cus;
        const int tiles_per_wave = per_cu >= 128 ? large_tiles_per_wave(lg.variant, per_cu)
                                                 : (int)std::max<int64_t>(1, std::min<int64_t>(4, per_cu / 16));
        const int64_t waves = (acc + tiles_per_wave - 1) / tiles_per_wave;
        sl.grid[g] = (waves + kWavesPerGroup - 1) / kWavesPerGroup;
        if (sl.grid[g] > 0x7fffffff)
            return set_error(AW4_EINVAL, "aw4_fused_step: %lld tiles exceed one launch", (long long)acc);
        h->count = n;
        h->cb1 = lg.cb1; h->lut1 = lg.lut1; h->cb2 = lg.cb2; h->lut2 = lg.lut2;
        h->total_tiles = acc;
        h->tiles_per_wave = tiles_per_wave;
    }
    return AW4_OK;
}

// One step kernel launch of a call that has made `launched` of them: a failure after the first
// is AW4_ELAUNCHED (the step's tensors may be partly updated).  aw4_inject_launch_failure makes
// the launch fail here without attempting it.
int launch_one(const void* fn, unsigned grid, void** args, hipStream_t s, int& launched) {
    const int code = launched > 0 ? AW4_ELAUNCHED : AW4_EHIP;
    if (g_fail_after >= 0 && launched >= g_fail_after) {
        g_fail_after = -1;
        return set_error(code, "step kernel launch %d: failure injected by aw4_inject_launch_failure", launched + 1);
    }
    const hipError_t err = hipLaunchKernel(fn, dim3(grid), dim3(kThreads), args, 0, s);
    if (err != hipSuccess)
        return set_error(code, "step kernel launch %d: %s%s", launched + 1, hipGetErrorString(err),
                         launched > 0 ? " (earlier launches of this step were enqueued)" : "");
    ++launched;
    return AW4_OK;
}

// Launch every group whose table is at dev_base + offset.
int launch_step(const StepLaunch& sl, const char* dev_base, const Tables* tables, hipStream_t s, int& launched) {
    for (size_t g = 0; g < sl.plan.size(); ++g) {
        if (sl.grid[g] == 0) continue;
        const StepHeader* dh = (const StepHeader*)(dev_base + sl.offset[g]);
        void* args[] = {(void*)&dh, (void*)&tables};
        const int rc = launch_one(kVariants[sl.plan[g].variant].fn, (unsigned)sl.grid[g], args, s, launched);
        if (rc) return rc;
    }
    return AW4_OK;
}

// Bytes of group g's launch table (header, rows, tile starts; without the 256-byte padding).
size_t group_table_bytes(const StepLaunch& sl, size_t g) {
    const size_t n = sl.plan[g].members.size();
    return sizeof(StepHeader) + sizeof(aw4_tensor) * n + sizeof(int64_t) * (n + 1);
}

// Whether every group can take its table in its launch's arguments.
bool fits_inline(const StepLaunch& sl) {
    for (size_t g = 0; g < sl.plan.size(); ++g)
        if (!kVariants[sl.plan[g].variant].fn_inline || group_table_bytes(sl, g) > (size_t)kInlineTableBytes)
            return false;
    return true;
}

// Launch every group with its table (at host + offset) in the launch's arguments.
int launch_step_inline(const StepLaunch& sl, const uint8_t* host, const Tables* tables, hipStream_t s) {
    InlineArgs a;
    a.tables = tables;
    a.reserved = 0;
    int launched = 0;
    for (size_t g = 0; g < sl.plan.size(); ++g) {
        if (sl.grid[g] == 0) continue;
        memcpy(a.table, host + sl.offset[g], group_table_bytes(sl, g));
        void* args[] = {(void*)&a};
        const int rc = launch_one(kVariants[sl.plan[g].variant].fn_inline, (unsigned)sl.grid[g], args, s, launched);
        if (rc) return rc;
    }
    return AW4_OK;
}

// Staging through kernel arguments: each launch carries up to kArgBytes of the table by value
// and copies them to their place in device memory, so the bytes need no device buffer of the
// host's and no copy engine, and the host's buffer is free again when the call returns (the
// launch packet holds its own copy).  Kernel arguments are limited to 4 KB per launch.
constexpr int kArgBytes = 3584;

struct __align__(16) ArgChunk {
    uint64_t dst;    // device address, 16-byte aligned
    uint32_t n16;    // 16-byte words to copy (at most kArgBytes / 16)
    uint32_t reserved;
    uint4 data[kArgBytes / 16];
};

__global__ void __launch_bounds__(256) stage_args_kernel(const ArgChunk chunk) {
    const uint4* src = (const uint4*)((const char*)__builtin_amdgcn_kernarg_segment_ptr() + offsetof(ArgChunk, data));
    for (uint32_t i = threadIdx.x; i < chunk.n16; i += 256) gaddr<u32x4>(chunk.dst)[i] = ((const u32x4*)src)[i];
}

int upload_by_arguments(const void* src, size_t bytes, uint8_t* dst, hipStream_t s) {
    ArgChunk chunk;
    for (size_t off = 0; off < bytes; off += kArgBytes) {
        const size_t n = std::min<size_t>(kArgBytes, bytes - off);
        memset(&chunk, 0, sizeof(chunk));
        chunk.dst = (uint64_t)(dst + off);
        chunk.n16 = (uint32_t)((n + 15) / 16);
        memcpy(chunk.data, (const char*)src + off, n);
        hipLaunchKernelGGL(stage_args_kernel, dim3(1), dim3(256), 0, s, chunk);
        AW4_HIP_CHECK(hipGetLastError());
    }
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
    StepLaunch sl;
    int rc = prepare_step(tensors, count, sl);
    if (rc || sl.plan.empty()) return rc;
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceState* ds = nullptr;
    rc = device_state(&ds);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    if (fits_inline(sl)) {
        std::vector<uint8_t>& host = ds->inline_host;
        host.resize(sl.bytes);
        rc = fill_step_tables(tensors, sl, ds->num_cus, host.data());
        if (rc) return rc;
        return launch_step_inline(sl, host.data(), ds->tables, s);
    }
    StagingSlot* sp = nullptr;
    rc = acquire_slot(ds, sl.bytes, &sp);
    if (rc) return rc;
    StagingSlot& slot = *sp;
    rc = fill_step_tables(tensors, sl, ds->num_cus, slot.host);
    if (rc) return rc;
    rc = upload_slot(slot, sl.bytes, s);
    if (rc) return rc;
    int launched = 0;
    rc = launch_step(sl, (const char*)slot.dev, ds->tables, s, launched);
    // the slot is in use by whatever was enqueued: it is not reused before that completes
    const hipError_t err = hipEventRecord(slot.done, s);
    slot.pending = err == hipSuccess;
    if (rc) return rc;
    if (err != hipSuccess)
        return set_error(AW4_ELAUNCHED, "hipEventRecord after the step's launches: %s", hipGetErrorString(err));
    return AW4_OK;
}

int aw4_fused_step_noalloc(const aw4_tensor* tensors, int32_t count, void* stream) {
    g_error.clear();
    StepLaunch sl;
    int rc = prepare_step(tensors, count, sl);
    if (rc || sl.plan.empty()) return rc;
    if (sl.bytes > (size_t)AW4_NOALLOC_TABLE_BYTES)
        return set_error(AW4_EINVAL,
                         "aw4_fused_step_noalloc: the launch tables of %d tensors need %zu bytes, more than its "
                         "%d-byte table area (use aw4_fused_step)",
                         count, sl.bytes, AW4_NOALLOC_TABLE_BYTES);
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceState* ds = nullptr;
    rc = device_state(&ds);
    if (rc) return rc;
    std::vector<uint8_t>& host = ds->noalloc_host;
    host.assign(sl.bytes, 0);
    rc = fill_step_tables(tensors, sl, ds->num_cus, host.data());
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    rc = upload_by_arguments(host.data(), sl.bytes, ds->scratch, s);
    if (rc) return rc;
    int launched = 0;
    return launch_step(sl, (const char*)ds->scratch, ds->tables, s, launched);
}

void aw4_inject_launch_failure(int32_t after) { g_fail_after = after < 0 ? -1 : after; }

int aw4_quantize(const float* values, int64_t numel, const aw4_moment* m, void* stream) {
    g_error.clear();
    if (!values || !m || numel <= 0 || numel % kBlock != 0)
        return set_error(AW4_EINVAL, "aw4_quantize: bad arguments (numel %lld)", (long long)numel);
    if (((uint64_t)values) % 16 != 0) return set_error(AW4_EALIGN, "aw4_quantize: values not 16-byte aligned");
    if (m->rounding == AW4_ROUND_FP32) return set_error(AW4_EINVAL, "aw4_quantize: fp32 moment");
    if (m->rounding == AW4_ROUND_LOOKAHEAD_SR)
        return set_error(AW4_EINVAL, "aw4_quantize: lookahead update-SR reads gradients (fused step only)");
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
                       *m, (const Tables*)ds->tables);
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

}  // extern "C"

namespace {

// The norm pass and coefficient of aw4_clip_coefficient (inv_scale null) and
// aw4_unscale_clip_coefficient.
int norm_prologue(const char* what, const aw4_tensor* tensors, int32_t count, const float* inv_scale,
                  float max_norm, float* norm_out, float* coef_out, float* found_out, void* stream) {
    g_error.clear();
    const bool unscale = inv_scale != nullptr;
    if (count <= 0 || !tensors || !norm_out || !coef_out || (unscale && !found_out))
        return set_error(AW4_EINVAL, "%s: bad arguments", what);
    if (!aligned((uint64_t)norm_out, 4) || !aligned((uint64_t)coef_out, 4) ||
        (unscale && (!aligned((uint64_t)inv_scale, 4) || !aligned((uint64_t)found_out, 4))))
        return set_error(AW4_EALIGN, "%s: device floats not 4-byte aligned", what);
    int result_dtype = tensors[0].grad_dtype;
    int64_t segments = 0;
    for (int i = 0; i < count; ++i) {
        const aw4_tensor& t = tensors[i];
        if (!t.grad || t.numel <= 0) return set_error(AW4_EINVAL, "tensor %d: null grad or numel %lld", i,
                                                      (long long)t.numel);
        if (t.grad_dtype != AW4_F32 && t.grad_dtype != AW4_BF16 && t.grad_dtype != AW4_F16)
            return set_error(AW4_EINVAL, "tensor %d: grad dtype %d", i, t.grad_dtype);
        if ((t.flags & AW4_TENSOR_VEC_ALIGNED) && !aligned(t.grad, t.grad_dtype == AW4_F32 ? 16 : 8))
            return set_error(AW4_EALIGN, "tensor %d: VEC_ALIGNED but grad misaligned", i);
        if (t.grad_dtype != result_dtype) result_dtype = AW4_F32;  // torch.stack promotes mixed dtypes
        segments += (t.numel + kNormSegment - 1) / kNormSegment;
    }
    if (segments > 0x7fffffff) return set_error(AW4_EINVAL, "%s: too many segments", what);
    // staging: header, rows, segment starts (copied), then the partial sums, the per-gradient
    // squared norms and (unscaling) the per-segment non-finite flags (device only)
    const size_t table = (sizeof(NormHeader) + sizeof(aw4_tensor) * count + sizeof(int64_t) * (count + 1) + 255) &
                         ~(size_t)255;
    const size_t bytes = table + sizeof(double) * ((size_t)segments + (size_t)count) +
                         (unscale ? sizeof(uint32_t) * (size_t)segments : 0);

    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceState* ds = nullptr;
    int rc = device_state(&ds);
    if (rc) return rc;
    StagingSlot* slot = nullptr;
    rc = acquire_slot(ds, bytes, &slot);
    if (rc) return rc;
    NormHeader* h = (NormHeader*)slot->host;
    memset(h, 0, sizeof(*h));
    aw4_tensor* rows = (aw4_tensor*)(h + 1);
    int64_t* starts = (int64_t*)(rows + count);
    int64_t acc = 0;
    for (int i = 0; i < count; ++i) {
        rows[i] = tensors[i];
        starts[i] = acc;
        acc += (tensors[i].numel + kNormSegment - 1) / kNormSegment;
    }
    starts[count] = acc;
    h->count = count;
    h->result_dtype = result_dtype;
    h->max_norm = max_norm;
    h->unscale = unscale ? 1 : 0;
    h->total_segments = segments;
    h->partials = (uint64_t)slot->dev + table;
    h->norm_sq = h->partials + sizeof(double) * (uint64_t)segments;
    h->norm_out = (uint64_t)norm_out;
    h->coef_out = (uint64_t)coef_out;
    if (unscale) {
        h->inv_scale = (uint64_t)inv_scale;
        h->nonfinite = h->norm_sq + sizeof(double) * (uint64_t)count;
        h->found_out = (uint64_t)found_out;
    }
    hipStream_t s = (hipStream_t)stream;
    rc = upload_slot(*slot, table, s);
    if (rc) return rc;
    const NormHeader* dh = (const NormHeader*)slot->dev;
    hipLaunchKernelGGL(norm_partials_kernel, dim3((unsigned)segments), dim3(kNormThreads), 0, s, dh);
    AW4_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(norm_tensor_kernel, dim3((unsigned)count), dim3(64), 0, s, dh);
    AW4_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(norm_finish_kernel, dim3(1), dim3(kNormThreads), 0, s, dh);
    AW4_HIP_CHECK(hipGetLastError());
    AW4_HIP_CHECK(hipEventRecord(slot->done, s));
    slot->pending = true;
    return AW4_OK;
}

}  // namespace

extern "C" {

int aw4_clip_coefficient(const aw4_tensor* tensors, int32_t count, float max_norm, float* norm_out,
                         float* coef_out, void* stream) {
    return norm_prologue("aw4_clip_coefficient", tensors, count, nullptr, max_norm, norm_out, coef_out, nullptr,
                         stream);
}

int aw4_unscale_clip_coefficient(const aw4_tensor* tensors, int32_t count, const float* inv_scale, float max_norm,
                                 float* norm_out, float* coef_out, float* found_inf_out, void* stream) {
    if (!inv_scale) return set_error(AW4_EINVAL, "aw4_unscale_clip_coefficient: null inv_scale");
    return norm_prologue("aw4_unscale_clip_coefficient", tensors, count, inv_scale, max_norm, norm_out, coef_out,
                         found_inf_out, stream);
}

int aw4_uniforms(uint64_t seed, uint64_t offset, int64_t n, float* out, void* stream) {
    g_error.clear();
    if (!out || n < 0 || offset > UINT64_MAX - (uint64_t)n) return set_error(AW4_EINVAL, "aw4_uniforms: bad arguments");
    if (n == 0) return AW4_OK;
    const int64_t lanes = (int64_t)(((offset + (uint64_t)n - 1) >> 7) - (offset >> 7) + 1) * 8;
    int64_t groups = (lanes + kThreads - 1) / kThreads;
    if (groups > 4096) groups = 4096;
    hipLaunchKernelGGL(uniforms_kernel, dim3((unsigned)groups), dim3(kThreads), 0, (hipStream_t)stream, seed, offset,
                       n, out);
    AW4_HIP_CHECK(hipGetLastError());
    return AW4_OK;
}

}  // extern "C"

#endif  // AW4_SCHED_ILP_TU
