// The step's prologue: the global gradient norm and clipping coefficient of
// torch.nn.utils.clip_grad_norm_ (norm type 2), which the reference's training examples
// run before every step (an HF Trainer with max_grad_norm=1.0,
// examples/train_gpt_small.py:214), optionally of the gradients GradScaler.unscale_ would leave
// (the loss scale's inverse applied in the same read).  One pass over the gradients: each
// workgroup sums the squares of one segment of one gradient in float64; one wave per gradient
// then combines its segments, and a single workgroup adds the per-gradient squares, both in a
// fixed order, with torch's rounding points (clip_grad.py _get_total_norm /
// _clip_grads_with_norm_):
//   g'     = grad_dtype(fp32(g * u))                   (unscaling: _amp_foreach_non_finite_check_and_unscale_)
//   norm_t = grad_dtype(fp32(sqrt(sum of g'^2)))       (torch._foreach_norm)
//   total  = R(fp32(sqrt(sum_t norm_t^2)))             (vector_norm of the stacked norms)
//   coef   = min(R(R(1 / R(total + 1e-6)) * max_norm), 1)
// with R the promotion of the gradient dtypes and every operation in fp32 rounded to R; with
// unscaling, found_inf = 1 if any g (the scaled value, as torch checks it) is not finite.  The
// unscaling and the coefficient are applied by the step itself (AW4_TENSOR_GRAD_UNSCALE,
// AW4_TENSOR_GRAD_SCALE), so neither the unscaled nor the clipped gradients are written.
#pragma once

#include "aw4_step.h"

namespace aw4 {

constexpr int kNormThreads = 256;
constexpr int64_t kNormSegment = 1 << 18;  // gradient values per workgroup of the norm pass

struct NormHeader {
    int32_t count;
    int32_t result_dtype;  // R
    float max_norm;
    int32_t unscale;       // nonzero: unscale by *inv_scale, and report found_inf
    int64_t total_segments;
    uint64_t partials;     // device address, double[total_segments]
    uint64_t norm_sq;      // device address, double[count]: norm_t^2 of each gradient
    uint64_t norm_out;     // device address, float
    uint64_t coef_out;     // device address, float
    uint64_t inv_scale;    // device address, float u (unscale)
    uint64_t nonfinite;    // device address, uint32[total_segments]: a segment holds a non-finite g (unscale)
    uint64_t found_out;    // device address, float found_inf (unscale)
};
// followed by aw4_tensor rows[count] and int64_t seg_start[count + 1]

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// One gradient value's contribution: its square, after unscaling (kUnscale: g' = G(fp32(g * u)),
// with a non-finite g recorded in `bad`, as torch checks the scaled value).
template <int G, bool kUnscale>
__device__ __forceinline__ double sq1(float f, float u, bool& bad) {
    if constexpr (kUnscale) {
        bad = bad | !__builtin_isfinite(f);
        f = round_to_dtype(f * u, G);
    }
    return (double)f * (double)f;
}

// Sum of squares of 4 consecutive gradient values starting at element e (all in range).
template <int G, bool kUnscale>
__device__ __forceinline__ double sq4(const aw4_tensor& T, int64_t e, bool vec, float u, bool& bad) {
    uint32_t w[4];
    float f[4];
    load_words<G>(T.grad, e, vec, w);
    words_to_f32<G>(w, f);
    double s = 0.0;
#pragma unroll
    for (int t = 0; t < 4; ++t) s += sq1<G, kUnscale>(f[t], u, bad);
    return s;
}

template <int G, bool kUnscale>
__device__ __forceinline__ double segment_sum(const aw4_tensor& T, int64_t e0, int64_t e1, bool vec, float u,
                                              bool& bad) {
    // Full groups of 4 values: thread i takes groups i, i + 256, ... (8 loads in flight per
    // thread: 4 KB per workgroup per load instruction).
    double acc = 0.0;
    const int64_t groups = (e1 - e0) >> 2;
    int64_t k = threadIdx.x;
    for (; k + 7 * kNormThreads < groups; k += 8 * kNormThreads) {
        double s[8];
#pragma unroll
        for (int v = 0; v < 8; ++v) s[v] = sq4<G, kUnscale>(T, e0 + 4 * (k + v * kNormThreads), vec, u, bad);
#pragma unroll
        for (int v = 0; v < 8; ++v) acc += s[v];
    }
    for (; k < groups; k += kNormThreads) acc += sq4<G, kUnscale>(T, e0 + 4 * k, vec, u, bad);
    // the tail of the tensor (fewer than 4 values)
    const int64_t tail = e0 + 4 * groups;
    if ((int64_t)threadIdx.x < e1 - tail) {
        float f;
        if (G == D_F32) f = gaddr<const float>(T.grad)[tail + threadIdx.x];
        else {
            const uint32_t h = gaddr<const uint16_t>(T.grad)[tail + threadIdx.x];
            f = G == D_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
        }
        acc += sq1<G, kUnscale>(f, u, bad);
    }
    return acc;
}

// One workgroup per segment: the float64 sum of squares of values
// [s * kNormSegment, min((s + 1) * kNormSegment, numel)) of one gradient -> partials[seg].
__global__ void __launch_bounds__(kNormThreads) norm_partials_kernel(const NormHeader* hdr) {
    const aw4_tensor* rows = (const aw4_tensor*)(hdr + 1);
    const int count = hdr->count;
    const int64_t* seg_start = (const int64_t*)(rows + count);
    const int64_t seg = blockIdx.x;
    const int t = tensor_of(seg_start, 0, count, seg);
    const aw4_tensor& T = rows[t];
    const int64_t e0 = (seg - seg_start[t]) * kNormSegment;
    const int64_t e1 = min(e0 + kNormSegment, T.numel);
    const bool vec = (T.flags & AW4_TENSOR_VEC_ALIGNED) != 0;
    double acc;
    bool bad = false;
    if (hdr->unscale) {
        const float u = *gaddr<const float>(hdr->inv_scale);
        if (T.grad_dtype == D_F32) acc = segment_sum<D_F32, true>(T, e0, e1, vec, u, bad);
        else if (T.grad_dtype == D_BF16) acc = segment_sum<D_BF16, true>(T, e0, e1, vec, u, bad);
        else acc = segment_sum<D_F16, true>(T, e0, e1, vec, u, bad);
    } else {
        if (T.grad_dtype == D_F32) acc = segment_sum<D_F32, false>(T, e0, e1, vec, 1.0f, bad);
        else if (T.grad_dtype == D_BF16) acc = segment_sum<D_BF16, false>(T, e0, e1, vec, 1.0f, bad);
        else acc = segment_sum<D_F16, false>(T, e0, e1, vec, 1.0f, bad);
    }
    acc = wave_sum_f64(acc);
    const bool wave_bad = __builtin_amdgcn_ballot_w64(bad) != 0;
    __shared__ double wave_acc[kNormThreads / 64];
    __shared__ uint32_t wave_bad_any[kNormThreads / 64];
    if ((threadIdx.x & 63) == 0) {
        wave_acc[threadIdx.x >> 6] = acc;
        wave_bad_any[threadIdx.x >> 6] = wave_bad ? 1u : 0u;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double s = wave_acc[0];
        uint32_t b = wave_bad_any[0];
#pragma unroll
        for (int w = 1; w < kNormThreads / 64; ++w) {
            s += wave_acc[w];
            b |= wave_bad_any[w];
        }
        gaddr<double>(hdr->partials)[seg] = s;
        if (hdr->unscale) gaddr<uint32_t>(hdr->nonfinite)[seg] = b;
    }
}

// One wave per gradient t: norm_sq[t] = norm_t^2 from its segments (lanes stride over them).
__global__ void __launch_bounds__(64) norm_tensor_kernel(const NormHeader* hdr) {
    const aw4_tensor* rows = (const aw4_tensor*)(hdr + 1);
    const int count = hdr->count;
    const int64_t* seg_start = (const int64_t*)(rows + count);
    const gptr<const double> partials = gaddr<const double>(hdr->partials);
    const int t = blockIdx.x;
    double s = 0.0;
    for (int64_t k = seg_start[t] + threadIdx.x; k < seg_start[t + 1]; k += 64) s += partials[k];
    s = wave_sum_f64(s);
    if (threadIdx.x == 0) {
        const float norm_t = round_to_dtype((float)__builtin_sqrt(s), rows[t].grad_dtype);
        gaddr<double>(hdr->norm_sq)[t] = (double)norm_t * (double)norm_t;  // exact
    }
}

// One workgroup: thread i adds norm_sq[i], norm_sq[i + 256], ...; the sums of the 4 waves are
// added in order; then the total norm and the coefficient.
__global__ void __launch_bounds__(kNormThreads) norm_finish_kernel(const NormHeader* hdr) {
    const int count = hdr->count;
    const gptr<const double> norm_sq = gaddr<const double>(hdr->norm_sq);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    double sq = 0.0;
    for (int t = threadIdx.x; t < count; t += kNormThreads) sq += norm_sq[t];
    sq = wave_sum_f64(sq);
    uint32_t bad = 0;
    if (hdr->unscale) {
        const gptr<const uint32_t> nonfinite = gaddr<const uint32_t>(hdr->nonfinite);
        for (int64_t k = threadIdx.x; k < hdr->total_segments; k += kNormThreads) bad |= nonfinite[k];
    }
    const bool wave_bad = __builtin_amdgcn_ballot_w64(bad != 0) != 0;
    __shared__ double wave_sq[kNormThreads / 64];
    __shared__ uint32_t wave_bad_any[kNormThreads / 64];
    if (lane == 0) {
        wave_sq[wave] = sq;
        wave_bad_any[wave] = wave_bad ? 1u : 0u;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double s = wave_sq[0];
#pragma unroll
        for (int w = 1; w < kNormThreads / 64; ++w) s += wave_sq[w];
        if (hdr->unscale) {
            uint32_t b = 0;
#pragma unroll
            for (int w = 0; w < kNormThreads / 64; ++w) b |= wave_bad_any[w];
            *gaddr<float>(hdr->found_out) = b ? 1.0f : 0.0f;
        }
        const int R = hdr->result_dtype;
        const float total = round_to_dtype((float)__builtin_sqrt(s), R);
        const float shifted = round_to_dtype(total + 1e-6f, R);
        const float inv = round_to_dtype(div_cr(1.0f, shifted), R);
        float coef = round_to_dtype(inv * hdr->max_norm, R);
        coef = coef > 1.0f ? 1.0f : coef;  // torch.clamp(max=1): NaN stays NaN
        *gaddr<float>(hdr->norm_out) = total;
        *gaddr<float>(hdr->coef_out) = coef;
    }
}

}  // namespace aw4
