/*
 * adamw4bit_hip.h -- C ABI of the MI355X (gfx950) fused 4-bit AdamW step.
 *
 * The library (libadamw4bit_hip.so) exports plain-C entry points that take
 * device addresses, sizes and a HIP stream.  No torch types cross this
 * boundary: the Python host code passes tensor data pointers and the
 * current stream handle through ctypes, exactly as a cgo/JNI/N-API binding
 * would.
 *
 * Reference interfaces replaced (nubank/adamw4bit, paths under src/adamw4bit/):
 *   aw4_fused_step   -> OptimizedBackend._step_parameter + _step_chunk
 *                       (_optimized.py:145-234) for EVERY parameter of one
 *                       optimizer.step() in a single launch; also the
 *                       element arithmetic of the reference step
 *                       QuantizedAdamW.step (adamw.py:547-803) for the
 *                       scheme set it shares with the optimized path.
 *   aw4_quantize     -> _optimized_quantization.quantize (:46-88) followed by
 *                       pack_4bit_codes (quantization.py:627-638) and the
 *                       in-place copy of MomentBuffer.write (_moment_buffer.py:164-179).
 *   aw4_dequantize   -> _optimized_quantization.dequantize (:91-107) on packed
 *                       codes (MomentBuffer.read, _moment_buffer.py:157-162).
 *
 * All entry points return 0 on success and a negative AW4_E* code on error;
 * aw4_last_error() then describes the failure (thread-local string).
 */
#ifndef ADAMW4BIT_HIP_H
#define ADAMW4BIT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AW4_ABI_VERSION 7
#define AW4_BLOCK 128 /* values per block scale (quantization.py:694-703, 4-bit default) */

/* Error codes. */
#define AW4_OK 0
#define AW4_EINVAL -1  /* malformed descriptor (null pointer, bad enum, bad size) */
#define AW4_EHIP -2    /* a HIP runtime call failed */
#define AW4_EALIGN -3  /* a buffer violates the alignment its descriptor promises */
/* A step failed after some of its step kernels were enqueued: parameters and
 * moment state may be partly updated (every other error enqueues no step
 * kernel, so the caller's tensors are unchanged). */
#define AW4_ELAUNCHED -4

/* 16-level codebooks (quantization.py:201-237, 401-422, 457-497). */
#define AW4_CB_NF4 0     /* nf4, nf4_sr */
#define AW4_CB_SDYN4 1   /* sdyn4, sdyn4_sr */
#define AW4_CB_DYN4 2    /* dyn4, dyn4_sr, dyn4_nz, dyn4_upd_sr_fp32read, dyn4_lookahead_sr, ..._nextbc */
#define AW4_CB_LIN4 3    /* lin4, lin4_sr, lin4_upd_sr_fp32read */
#define AW4_CB_LIN4_NZ 4 /* lin4_nz */
#define AW4_NUM_CODEBOOKS 5

/* How a moment is stored and re-encoded. */
#define AW4_ROUND_FP32 0      /* fp32 state tensor, no codec (adamw.py:807-817 ineligible or "fp32") */
#define AW4_ROUND_RTN 1       /* nearest level, ties up (_compiled_quantization.py:41-45) */
#define AW4_ROUND_STATE_SR 2  /* value-unbiased SR (_compiled_quantization.py:60-71) */
#define AW4_ROUND_UPDATE_SR 3 /* preconditioner-space SR (_compiled_quantization.py:74-109) */
/* m2 only, dyn4 codebook: lookahead update-SR (quantize_dyn4_la_upd_sr,
 * quantization.py:779-895).  The probability is computed in float64 on the next
 * step's preconditioner beta2 * q + fresh, fresh = (1-beta2) * g^2, from the
 * aw4_moment la_* constants; the uniforms are float64.  Stores codes and scales
 * (dyn4_proxy_la_upd_sr, dyn4_vproxy_la_upd_sr, adamw.py:579-614), or, with
 * AW4_MOMENT_PENDING, samples the fp32 pending state before the update instead
 * (dyn4_la_upd_sr, adamw.py:566-578). */
#define AW4_ROUND_LOOKAHEAD_SR 4

/* aw4_moment.flags */
#define AW4_MOMENT_ZERO_FLOOR 0x1 /* code 0 -> code 1 after rounding (dyn4_nz, quantization.py:529-552) */
#define AW4_MOMENT_EDEN 0x2       /* EDEN block-scale calibration (_optimized_quantization.py:81-85) */
#define AW4_MOMENT_GUARDS 0x4     /* exact-level SR guards of the optimized path (_compiled_quantization.py:48-57);
                                     clear for the reference step (quantization.py:279-377) */
#define AW4_MOMENT_EXT_DRAWS 0x8  /* read uniforms from aw4_moment.draws instead of on-device Philox */
/* m2 only: the parameter update's denominator reads the value just stored,
 * cb[code] * scale, instead of the fp32 lerp (dyn4_upd_sr / lin4_upd_sr,
 * adamw.py:636-656, quantization.py:748-776).  If `values` is set it receives
 * 1 / denominator per element (m2_read_preconditioner, adamw.py:632). */
#define AW4_MOMENT_SAMPLED_READ 0x10
/* with AW4_MOMENT_SAMPLED_READ: read with the scale before the EDEN calibration
 * that AW4_MOMENT_EDEN applies to the stored scale (*_upd_sr_store_eden,
 * adamw.py:615-635, quantization.py:1007-1037) */
#define AW4_MOMENT_READ_RAW_SCALE 0x20
/* AW4_ROUND_LOOKAHEAD_SR: fresh = fp32(fp32(1-beta2) * m2) instead of (1-beta2) * g^2
 * (the v-proxy, dyn4_vproxy_la_upd_sr, adamw.py:597-614) */
#define AW4_MOMENT_FRESH_PROXY 0x40
/* AW4_ROUND_LOOKAHEAD_SR: `values` is the fp32 pending second moment z.  The step
 * samples z (codes are not kept) and sets m2 = fp32(beta2) * sample + (1-beta2) * g * g
 * (addcmul), then stores m2 back to `values` (dyn4_la_upd_sr, adamw.py:566-578, 771-776). */
#define AW4_MOMENT_PENDING 0x80

/* aw4_tensor.param_dtype / grad_dtype */
#define AW4_F32 0
#define AW4_BF16 1
#define AW4_F16 2
/* float64 (the reference's optimized backend takes float64 parameters, _optimized.py:99): the
 * gradient is read as fp32(g) (gradient.to(float32), _optimized.py:215), the moments and the
 * denominator are fp32 as for every dtype, and the parameter is updated in float64 with
 * decay_f64 and step_coef_f64.  Not with AW4_TENSOR_GRAD_SCALE / AW4_TENSOR_GRAD_UNSCALE. */
#define AW4_F64 3

/* aw4_tensor.flags */
#define AW4_TENSOR_LERP1_LARGE 0x1 /* lerp weight 1-beta1 >= 0.5: m1 = fma(w-1, g-m1, g) */
#define AW4_TENSOR_LERP2_LARGE 0x2 /* same for m2 with g*g */
#define AW4_TENSOR_VEC_ALIGNED 0x4 /* param and grad allow 4-element vector access */
/* `grad_scale` is the device address of a float pair {u, c}.  With AW4_TENSOR_GRAD_UNSCALE
 * every gradient value g is first read as grad_dtype(fp32(g * u)) (the unscaling of
 * GradScaler.unscale_, u its fp32 inverse loss scale; see aw4_unscale_clip_coefficient); with
 * AW4_TENSOR_GRAD_SCALE it is then read as grad_dtype(fp32(g * c)) (the gradient clipping of
 * torch.nn.utils.clip_grad_norm_, whose _foreach_mul_ rounds each product to the gradient's
 * dtype; see aw4_clip_coefficient).  The gradients in memory are not changed. */
#define AW4_TENSOR_GRAD_SCALE 0x8
#define AW4_TENSOR_GRAD_UNSCALE 0x10

/*
 * One moment (m1 or m2) of one parameter.  For a quantized moment, `codes`
 * holds ceil(numel/2) bytes (element 2j in the low nibble of byte j) and
 * `scales` numel/128 fp32 block scales; `values` is 0, or, for an m2 with
 * AW4_MOMENT_SAMPLED_READ, the numel fp32 outputs of 1 / denominator.  For an
 * fp32-state moment only `values` (numel fp32) is set.  Layout as in
 * optimizer.state (_moment_buffer.py:89-142, adamw.py:326-362).
 */
typedef struct aw4_moment {
    uint64_t codes;      /* device address, uint8[ceil(numel/2)], 8-byte aligned, or 0 */
    uint64_t scales;     /* device address, float[numel/128] or 0 */
    uint64_t values;     /* device address, float[numel] (fp32 state, or SAMPLED_READ output) or 0 */
    uint64_t draws;      /* device address of numel uniforms (AW4_MOMENT_EXT_DRAWS): float, double for
                            AW4_ROUND_LOOKAHEAD_SR; or 0 */
    uint64_t rng_seed;   /* Philox4x32-10 key: generator seed of this moment's stream */
    uint64_t rng_offset; /* stream position of this write's first draw; multiple of 128 */
    int32_t codebook;    /* AW4_CB_* (ignored for AW4_ROUND_FP32) */
    int32_t rounding;    /* AW4_ROUND_* */
    int32_t flags;       /* AW4_MOMENT_* */
    float sr_bias;       /* update-SR storage bias correction, fp32(max(c,1e-12)) (_optimized_quantization.py:66-67) */
    float sr_bias_rcp;   /* correctly rounded 1/sr_bias */
    float sr_eps;        /* update-SR epsilon, fp32(eps) */
    /* AW4_ROUND_LOOKAHEAD_SR, as the float64 values the reference computes with:
     * beta2, 1.0 - beta2, max(bias_correction, 1e-12), eps */
    double la_beta2;
    double la_fresh_weight;
    double la_bias;
    double la_eps;
} aw4_moment; /* 104 bytes */

/*
 * One parameter of a step.  All scalars are the fp32 values the reference's
 * ATen kernels see (_optimized.py:168-173, :215-222):
 *   w1 = fp32(1-beta1) (or fp32(1-beta1) - 1 with LERP1_LARGE), w2 likewise,
 *   decay = fp32(1 - lr*wd), step_coef = fp32(-lr/bc1),
 *   bc2_sqrt = fp32(sqrt(bc2)), bc2_sqrt_rcp = RN(1/bc2_sqrt), eps = fp32(eps);
 * and for an AW4_F64 parameter the float64 values themselves:
 *   decay_f64 = 1 - lr*wd, step_coef_f64 = -lr/bc1
 * (p = p * decay_f64, then p = p + (step_coef_f64 * m1) / den in float64, _optimized.py:221-222).
 */
typedef struct aw4_tensor {
    uint64_t param;      /* device address, contiguous, param_dtype[numel]; updated in place */
    uint64_t grad;       /* device address, contiguous, grad_dtype[numel] */
    uint64_t grad_scale; /* device address of the float pair {u, c} (AW4_TENSOR_GRAD_UNSCALE /
                            AW4_TENSOR_GRAD_SCALE) or 0 */
    int64_t numel;
    int32_t param_dtype; /* AW4_F32 / AW4_BF16 / AW4_F16 / AW4_F64 */
    int32_t grad_dtype;
    int32_t flags;       /* AW4_TENSOR_* */
    float w1, w2, decay, step_coef, bc2_sqrt, bc2_sqrt_rcp, eps;
    aw4_moment m1;
    aw4_moment m2;
    double decay_f64, step_coef_f64; /* AW4_F64 parameters (else unused) */
} aw4_tensor; /* 296 bytes */

/* Library ABI version (AW4_ABI_VERSION of the build). */
int aw4_abi_version(void);

/* Description of the last error on this thread ("" if none). */
const char* aw4_last_error(void);

/*
 * One fused AdamW step over `count` parameters on `stream` (a hipStream_t;
 * 0 = legacy default stream): one kernel launch per group of parameters that
 * share a kernel (one launch for a recipe's parameters).  `tensors` is a host
 * array: a group of up to 11 parameters on the ZE-EDEN or ZIP-SR kernels
 * receives its rows in its launch's arguments, any other step's rows are
 * staged to device memory by the library (the call returns before the step
 * completes, stream-ordered like any HIP launch).
 * Replaces the per-parameter chunk loop of _optimized.py:145-203 and the
 * chunk update _optimized.py:206-234.
 */
int aw4_fused_step(const aw4_tensor* tensors, int32_t count, void* stream);

/*
 * aw4_fused_step for callers that cannot allocate device memory: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  It has no counterpart in
 * the reference (whose step is Python).  Same arguments, checks, kernels and results as
 * aw4_fused_step, but it calls no hipMalloc, hipFree or other allocating routine: the launch
 * tables (the step's only device memory besides the caller's tensors) go to a fixed area of
 * AW4_NOALLOC_TABLE_BYTES that the library holds in a file-scope device array on each GPU
 * until the process ends, and reach it through the arguments of small copy kernels on
 * `stream`.  A call whose tables exceed that area (about 3,400 tensors) fails with AW4_EINVAL.
 * The first call on a device (of any entry point) copies the codebook tables to it once,
 * synchronously.  Every call on one GPU uses the same area: calls on one stream are ordered,
 * calls that overlap on different streams of one GPU race.
 */
#define AW4_NOALLOC_TABLE_BYTES (1 << 20)
int aw4_fused_step_noalloc(const aw4_tensor* tensors, int32_t count, void* stream);

/*
 * For tests of a caller's error handling; no counterpart in the reference.  The
 * next aw4_fused_step or aw4_fused_step_noalloc call on this thread makes
 * `after` step kernel launches and then fails as a failed launch would
 * (AW4_ELAUNCHED if `after` > 0, else AW4_EHIP): the launch is not made, so no
 * device fault is involved.  A negative `after` clears it.
 */
void aw4_inject_launch_failure(int32_t after);

/*
 * Encode `numel` fp32 values (numel a multiple of 128) into the quantized
 * moment `m` (codes + scales written in place), with m's rounding, codebook,
 * flags and draws.  Replaces _optimized_quantization.quantize (:46-88) +
 * pack_4bit_codes.  `values` is a device address.
 */
int aw4_quantize(const float* values, int64_t numel, const aw4_moment* m, void* stream);

/*
 * Decode a quantized moment into fp32 `out` (device address, numel values,
 * numel a multiple of 128).  Replaces _optimized_quantization.dequantize (:91-107).
 */
int aw4_dequantize(const aw4_moment* m, int64_t numel, float* out, void* stream);

/*
 * Fill `out` (device address, n floats) with the uniforms in [0,1) that a
 * stochastic write draws at stream positions offset .. offset+n-1 of the
 * Philox4x32-10 stream keyed by `seed`.  Positions are grouped by 128: position
 * P = 128 B + 32 q + 4 j + t (q, t in 0..3, j in 0..7) is the 24-bit field
 * 4 q + t of the 384-bit little-endian string formed by the outputs of
 * Philox(counter = 24 B + 3 j + r, key = seed), r = 0, 1, 2, times 2^-24.  Draw
 * k of a write of moment m is the uniform at position m.rng_offset + k, k being
 * the element index; it replaces _optimized_quantization._uniform_draws
 * (:37-43), whose CPU mt19937 / CUDA Philox streams a device kernel cannot
 * reproduce.
 */
int aw4_uniforms(uint64_t seed, uint64_t offset, int64_t n, float* out, void* stream);

/*
 * The global gradient clipping that precedes step() in the reference's training
 * examples (an HF Trainer with max_grad_norm=1.0, examples/train_gpt_small.py:214),
 * i.e. torch.nn.utils.clip_grad_norm_(params, max_norm) (norm type 2), computed on
 * device in one pass over the gradients of `count` rows (grad, grad_dtype, numel and
 * AW4_TENSOR_VEC_ALIGNED are read; every other field is ignored):
 *   norm_t = ||grad_t||_2 rounded to grad_t's dtype (torch._foreach_norm),
 *   total  = sqrt(sum_t norm_t^2) rounded to R, the promotion of all gradient dtypes,
 *   coef   = min(RN(RN(1 / RN(total + 1e-6)) * max_norm), 1), each op rounded to R
 *            (clip_grad.py: max_norm / (total_norm + 1e-6) is reciprocal then multiply).
 * Sums of squares are taken in float64 in a fixed order (the result does not depend on
 * the launch shape).  Writes the fp32 values of total to norm_out[0] and of coef to
 * coef_out[0] (device addresses) without a host synchronisation.  Put coef in the second
 * float of the rows' grad_scale pair (AW4_TENSOR_GRAD_SCALE) of the next aw4_fused_step: the
 * step then reads the clipped gradients the in-place _foreach_mul_ would have written, and
 * the gradients themselves stay unscaled in memory (no extra pass over them).
 */
int aw4_clip_coefficient(const aw4_tensor* tensors, int32_t count, float max_norm, float* norm_out,
                         float* coef_out, void* stream);

/*
 * The same pass over gradients that a GradScaler has scaled: GradScaler.unscale_
 * (torch/amp/grad_scaler.py, _amp_foreach_non_finite_check_and_unscale_) followed by
 * aw4_clip_coefficient, fused.  Each value is read once as g' = grad_dtype(fp32(g * u)),
 * u = the fp32 at device address inv_scale (GradScaler's fp32 1 / scale); the norm and
 * coefficient are those of aw4_clip_coefficient over the g', and found_inf_out[0] (device)
 * receives 1.0 if any g is not finite, else 0.0, torch's found_inf.  Nothing is written to
 * the gradients: put u and coef in the rows' grad_scale pair of the next aw4_fused_step with
 * AW4_TENSOR_GRAD_UNSCALE (and AW4_TENSOR_GRAD_SCALE to clip).  With max_norm = +inf it is
 * the unscaling and inf check alone (coef 1 for finite norms).  No counterpart in the
 * reference, whose examples scale no loss; its trainer's GradScaler path
 * (examples/train_gpt_small.py:214-215 via the HF Trainer) runs these as torch ops.
 */
int aw4_unscale_clip_coefficient(const aw4_tensor* tensors, int32_t count, const float* inv_scale, float max_norm,
                                 float* norm_out, float* coef_out, float* found_inf_out, void* stream);

/*
 * Host-only: copy the encode lookup tables the kernels use into `out`
 * (host memory, `bytes` long); returns the table size in bytes (call with
 * out = 0 to query) or a negative error.  Layout: for each of AW4_NUM_LUTS
 * tables, AW4_LUT_ENTRIES entries {float threshold; uint32 base; float
 * level_lo; float level_hi}: a value x in bucket k (bucket function below)
 * encodes to base + (x >= threshold); level_lo and level_hi are the levels
 * cb[min(code, 15)] of the two outcomes (round-to-nearest tables: the code's
 * level; level-count tables: the upper neighbour of x).
 * Tables 0..5: round-to-nearest codes for nf4, sdyn4, dyn4, lin4, lin4_nz,
 * dyn4 with the zero floor; tables 6..10: searchsorted-left counts
 * (number of levels < x) for nf4, sdyn4, dyn4, lin4, lin4_nz.
 * Bucket of x: a = bits(x) & 0x7fffffff; k = clamp((a >> 20) - AW4_LUT_EXP0 + 1,
 * 0, AW4_LUT_HALF - 1); bucket = k + (bits(x) >> 31) * AW4_LUT_HALF.
 */
#define AW4_NUM_LUTS 11
#define AW4_LUT_HALF 89
#define AW4_LUT_ENTRIES (2 * AW4_LUT_HALF)
#define AW4_LUT_EXP0 936 /* (127 - 10) << 3: |x| < 2^-10 shares bucket 0 */
int64_t aw4_encode_tables(void* out, int64_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* ADAMW4BIT_HIP_H */
