/*
 * CastForge MI355X quantized-weight hot path — C ABI (`include/castforge_hip.h`).
 *
 * Sits beside the unchanged `include/castforge.h` of sungdomo/CastForge and follows the
 * conventions of its FFI (src/ffi.rs:13-215, include/castforge.h:18-52):
 *   - every entry point returns int32_t: 0 success, 1 error (message in *out_error),
 *     2 internal exception caught; nothing throws or aborts across the ABI;
 *   - *out_error (may be NULL) is cleared on entry and, when set, is a heap string the caller
 *     frees with castforge_hip_free_string (ffi.rs:25-31);
 *   - the caller owns every buffer; the library allocates no device memory;
 *   - buffers named src/codes/scales/zeros/absmax/x/y are DEVICE pointers; `stream` is a
 *     hipStream_t (NULL = the null stream); work is enqueued asynchronously on it;
 *   - shapes are int64 element counts; weights are row-major [N, K] with K contiguous, the
 *     `packed_rhs` layout of the reference (passes/weights/fold.rs:549-554);
 *   - calls on different streams are independent; no global mutable state, except the
 *     per-device scratch array of castforge_hip_quantize_groupwise_noalloc.
 *
 * Packed formats (new in this library; the reference stores one i8 per element):
 *   INT8  : codes i8 [N, K]; scales f32 [N] (per channel) or [1] (per tensor).
 *   INT4g : codes u32 [N, K/8], element k in bits 4*(k%8); scales f16 bits [N, GP] with
 *           GP = 8*ceil(G/8) (each row padded to a 16-byte multiple, pad slots written 0);
 *           zeros u32 [N, ceil(G/8)], group g in bits 4*(g%8); G = ceil(K/group).
 *           dequant = (q - z) * f32(scale).
 *   NF4   : codes u32 [N, K/8] (same packing); absmax f32 [N, ceil(K/block)].
 *           dequant = NF4_TABLE[q] * absmax.
 *   FP8   : codes u8 [R, C] OCP E4M3FN; scales f32 [R]; dequant = e4m3(q) * scale.
 */
#ifndef CASTFORGE_HIP_H
#define CASTFORGE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CASTFORGE_HIP_ABI_VERSION 1
#define CFH_MAX_BATCH 8

/* Rounding rule of the integer quantizers.  HALF_AWAY is Rust's f32::round used by the
 * reference (formats.rs:676, schemes.rs:546); HALF_EVEN is IEEE round-to-nearest-even. */
enum { CFH_ROUND_HALF_AWAY = 0, CFH_ROUND_HALF_EVEN = 1 };
/* Scale granularity of the symmetric INT8/INT4 quantizer. */
enum { CFH_GRAN_TENSOR = 0, CFH_GRAN_CHANNEL = 1 };
/* Element types of activations / outputs. */
enum { CFH_DTYPE_F32 = 0, CFH_DTYPE_BF16 = 1 };

/* ---- library ---------------------------------------------------------------------------- */

/* Mirrors castforge_version (castforge.h:18-21, ffi.rs:13-23): static string, do not free. */
const char *castforge_hip_version(void);

/* Mirrors castforge_free_string (castforge.h:23-26, ffi.rs:25-31). NULL is ignored. */
void castforge_hip_free_string(char *ptr);

/* Device name, CU count, HBM size and arch of the current device as a JSON heap string. */
int32_t castforge_hip_device_info(char **out_json, char **out_error);

/* ---- quantize / dequantize --------------------------------------------------------------- */

/* Symmetric absmax quantization of f32 [rows, cols] to i8 codes.
 * Replaces quantize_symmetric_f32 (passes/quantize/formats.rs:664-698) as called by
 * QuantizeWeightsPass::run (passes/quantize/schemes.rs:324-452): amax = NaN-ignoring max |v|,
 * scale = amax < 1e-12 ? 1 : amax / qmax, q = clamp(round(v / scale), qmin, qmax), NaN -> 0;
 * bits == 4 -> [-8, 7], anything else -> [-128, 127] (formats.rs:654-660).
 * CFH_GRAN_TENSOR writes scales[0] (the reference); CFH_GRAN_CHANNEL writes scales[rows]. */
int32_t castforge_hip_quantize_int8(const float *src, int64_t rows, int64_t cols, int32_t bits,
                                    int32_t granularity, int32_t round_mode, int8_t *codes,
                                    float *scales, void *stream, char **out_error);

/* (q - 0) * scale to f32.  Replaces TensorStore::resolve_f32_attr for QuantizedI8
 * (ir/tensor_store.rs:323-331) and the evaluator's dequant (codegen/eval.rs:305-319). */
int32_t castforge_hip_dequantize_int8(const int8_t *codes, const float *scales, int64_t rows,
                                      int64_t cols, int32_t granularity, float *out, void *stream,
                                      char **out_error);

/* INT4 asymmetric group-wise along K, fp16 scale and u4 zero point, 8 codes per u32.
 * New scheme behind quantize(bits=4,group=..) (registry/families.rs:133-137); the reference's
 * group-wise pass (passes/quantize/schemes.rs:532-549) is symmetric and keeps no codes.
 * group: power of two in [8, 256]; cols % 8 == 0; src 16-byte aligned.
 * Per group: h = f16_rne((max - min) / 15) (range < 1e-12 -> 1.0; 0 -> 0x0001; Inf -> 0x7BFF),
 * s = f32(h), z = clamp(rne(-min / s), 0, 15), q = clamp(rne(v / s) + z, 0, 15), NaN -> z. */
int32_t castforge_hip_quantize_int4g(const float *src, int64_t rows, int64_t cols, int64_t group,
                                     uint32_t *codes, uint16_t *scales_f16, uint32_t *zeros,
                                     void *stream, char **out_error);

/* castforge_hip_quantize_int4g of the AWQ-style pre-scaled weight W'[n, k] = f32(W[n, k] *
 * in_scale[k]) (s = a^0.5 per input channel), fused into the same pass so
 * W' is never written.  in_scale: device f32 [cols], 16-byte aligned.  New; no reference
 * counterpart (the reference's "AWQ" is the salient halving of quantize-groupwise). */
int32_t castforge_hip_quantize_int4g_awq(const float *src, const float *in_scale, int64_t rows, int64_t cols,
                                         int64_t group, uint32_t *codes, uint16_t *scales_f16,
                                         uint32_t *zeros, void *stream, char **out_error);

int32_t castforge_hip_dequantize_int4g(const uint32_t *codes, const uint16_t *scales_f16,
                                       const uint32_t *zeros, int64_t rows, int64_t cols,
                                       int64_t group, float *out, void *stream, char **out_error);

/* NF4 block-wise along K (QLoRA normal-float table), f32 absmax per block, 8 codes per u32.
 * New scheme (claimed by the reference README.md:68, absent from its code).
 * block: power of two in [8, 512]; cols % 8 == 0.  stored = absmax < 1e-12 ? 1 : absmax;
 * code = #{i : v / stored > (T[i] + T[i+1]) / 2}, NaN -> 7. */
int32_t castforge_hip_quantize_nf4(const float *src, int64_t rows, int64_t cols, int64_t block,
                                   uint32_t *codes, float *absmax, void *stream, char **out_error);

int32_t castforge_hip_dequantize_nf4(const uint32_t *codes, const float *absmax, int64_t rows,
                                     int64_t cols, int64_t block, float *out, void *stream,
                                     char **out_error);

/* FP8 E4M3FN per row (weights: per output channel; activations: per token, dynamic):
 * scale = absmax < 1e-12 ? 1 : absmax / 448, code = f32_to_fp8_e4m3fn(v / scale) bit-exact
 * with the reference codec (passes/serving/mutable_loads.rs:367-411).  src_dtype F32 or BF16. */
int32_t castforge_hip_quantize_fp8(const void *src, int32_t src_dtype, int64_t rows, int64_t cols,
                                   uint8_t *codes, float *scales, void *stream, char **out_error);

/* fp8_e4m3fn_to_f32 (mutable_loads.rs:415-432) times the row scale. */
int32_t castforge_hip_dequantize_fp8(const uint8_t *codes, const float *scales, int64_t rows,
                                     int64_t cols, float *out, void *stream, char **out_error);

/* Group-wise symmetric write-back quantizer with AWQ salient protection.  Replaces
 * QuantizeGroupwisePass::run (passes/quantize/schemes.rs:456-630) on one tensor flattened to n
 * elements: chunks of max(group_size, 2) consecutive elements; scale = gmax < 1e-12 ? 1 :
 * gmax / qmax; salient elements (|v| >= the salient_count-th largest |v| in total order, with
 * salient_count = min(max(ceil(f32(n) * clamp(salient_ratio, 0.001, 0.5)), 1), n)) use half
 * the scale when awq_salient is set; deq = clamp(round(v / eff), qmin, qmax) * eff.
 * Writes deq (f32 [n]), the group scales (f32 [ceil(n / group)], may be NULL) and, when
 * salient_count_out is not NULL, the salient count (a host pointer).  The threshold search
 * needs a device workspace of CFH_GROUPWISE_WORKSPACE_BYTES (unused when awq_salient = 0). */
#define CFH_GROUPWISE_WORKSPACE_BYTES 2048
int32_t castforge_hip_quantize_groupwise(const float *src, int64_t n, int32_t bits, int64_t group_size,
                                         int32_t awq_salient, float salient_ratio, int32_t round_mode,
                                         float *deq, float *scales, void *workspace,
                                         int64_t *salient_count_out, void *stream, char **out_error);

/* No counterpart in the reference.  castforge_hip_quantize_groupwise for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the AWQ threshold search runs in a static per-device scratch array of
 * CFH_GROUPWISE_WORKSPACE_BYTES (held until the process ends) instead of a caller workspace,
 * and the call allocates nothing.  Same arguments and results otherwise; n < 2^32 (the limit
 * of the search's 32-bit counters), larger tensors are rejected with rc 1.  Every call on one
 * GPU shares that GPU's array and re-initialises it on its stream: calls that overlap on one
 * GPU (different streams or host threads) race and must be serialised by the caller. */
int32_t castforge_hip_quantize_groupwise_noalloc(const float *src, int64_t n, int32_t bits,
                                                 int64_t group_size, int32_t awq_salient,
                                                 float salient_ratio, int32_t round_mode, float *deq,
                                                 float *scales, int64_t *salient_count_out, void *stream,
                                                 char **out_error);

/* FP8 / MXFP8 uniform-grid write-back quantizer.  Replaces QuantizeFp8Pass::run
 * (passes/quantize/schemes.rs:633-754): blocks of max(block_size, 4) consecutive elements;
 * raw = amax < 1e-12 ? 1 : amax / fp8_max (448 E4M3, 57344 E5M2); scale = mxfp8 ?
 * powf(2, ceilf(log2f(raw))) (glibc's rounding of log2f reproduced exactly) : raw;
 * deq = round(clamp(v / scale, -max, max) / step) * step * scale with step = max / 31 (E4M3)
 * or max / 15 (E5M2), round half away from zero. */
int32_t castforge_hip_quantize_fp8_grid(const float *src, int64_t n, int32_t e5m2, int32_t mxfp8,
                                        int64_t block_size, float *deq, void *stream, char **out_error);

/* Several matrices in as few launches as possible: one per column count (at most 8 matrices,
 * and for INT4 at most 65535 rows, per launch), e.g. every projection of a decoder block.
 * Codes, scales and zero points are bit-identical to one castforge_hip_quantize_int4g /
 * castforge_hip_quantize_int8 (CFH_GRAN_CHANNEL) call per matrix, with the same validation;
 * a matrix the batched kernels cannot take (alignment, row length) is quantized on its own.
 * The reference's QuantizeWeightsPass quantizes every constant of the module in turn
 * (passes/quantize/schemes.rs:301-453); this is that loop in one or two launches. */
typedef struct cfh_quant_problem_t {
    const float *src;  /* f32 [rows, cols] */
    int64_t rows, cols;
    void *codes;       /* INT4: u32 [rows, cols/8]; INT8: i8 [rows, cols] */
    void *scales;      /* INT4: f16 [rows, GP]; INT8: f32 [rows] */
    uint32_t *zeros;   /* INT4: u32 [rows, ceil(G/8)]; INT8: unused */
} cfh_quant_problem_t;

int32_t castforge_hip_quantize_int4g_batched(const cfh_quant_problem_t *problems, int32_t count,
                                             int64_t group, void *stream, char **out_error);

/* castforge_hip_quantize_int4g_awq over up to CFH_MAX_BATCH matrices in as few launches as
 * castforge_hip_quantize_int4g_batched: in_scales is a host array of `count` device pointers,
 * in_scales[i] the f32 [cols] pre-scale of problem i (16-byte aligned).  New; no reference
 * counterpart (BASELINE config 5's per-layer AWQ quantize). */
int32_t castforge_hip_quantize_int4g_awq_batched(const cfh_quant_problem_t *problems,
                                                 const float *const *in_scales, int32_t count,
                                                 int64_t group, void *stream, char **out_error);

int32_t castforge_hip_quantize_int8_batched(const cfh_quant_problem_t *problems, int32_t count,
                                            int32_t bits, int32_t round_mode, void *stream,
                                            char **out_error);

/* ---- dequant-fused matmul ----------------------------------------------------------------- */
/* y[m, n] = sum_k x[m, k] * dequant(W)[n, k]; x bf16 [M, K]; y f32 or bf16 [M, N].
 * Replaces the evaluation of `castforge.fused_qmatmul` (passes/fuse/epilogue.rs:10-94,
 * codegen/eval.rs:1145-1179 -> eval_matmul_2d eval.rs:1465-1507, packed_rhs) and the HIP text
 * the reference emits for it (codegen/targets/gpu_c.rs:208-292, passes/loops/lower.rs:226-247).
 * M <= 64 (INT8: M <= 32) runs the MFMA decode / skinny kernels; larger M the prefill GEMM. */
int32_t castforge_hip_gemv_w4a16(const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t group,
                                 const uint32_t *codes, const uint16_t *scales_f16,
                                 const uint32_t *zeros, void *y, int32_t y_dtype, void *stream,
                                 char **out_error);

int32_t castforge_hip_gemv_w8a16(const uint16_t *x, int64_t m, int64_t n, int64_t k,
                                 const int8_t *codes, const float *scales, int32_t granularity,
                                 void *y, int32_t y_dtype, void *stream, char **out_error);

int32_t castforge_hip_gemv_nf4(const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t block,
                               const uint32_t *codes, const float *absmax, void *y, int32_t y_dtype,
                               void *stream, char **out_error);

/* Several W4A16 problems with the same M (1..64) in ONE launch, e.g. the 7 projections of a
 * decoder block; each needs k % 128 == 0, group % 128 == 0 and 16-byte aligned x / codes. */
typedef struct cfh_w4a16_problem_t {
    const uint16_t *x;          /* bf16 [M, k] */
    const uint32_t *codes;      /* u32 [n, k/8] */
    const uint16_t *scales_f16; /* f16 [n, GP] */
    const uint32_t *zeros;      /* u32 [n, ceil(G/8)] */
    void *y;                    /* [M, n] */
    int64_t n, k, group;
} cfh_w4a16_problem_t;

int32_t castforge_hip_gemv_w4a16_batched(const cfh_w4a16_problem_t *problems, int32_t count,
                                         int64_t m, int32_t y_dtype, void *stream,
                                         char **out_error);

/* GEMV planes: the layout of INT4 g128 weights that the M = 1 decode kernel below streams, built
 * once at load time (no reference counterpart: the reference keeps one i8 per element,
 * ir/tensor_store.rs:44-48).  For an [N, K] matrix (K % 128 == 0, group 128), T = ceil(N/16),
 * G = K/128:
 *   planes_codes : T x G chunks of 1024 bytes; chunk (t, g) holds, at byte 16 * (16 p + r),
 *                  canonical code words 16 g + 4 p .. 16 g + 4 p + 3 of row 16 t + r
 *                  (p = 0..3), so one wave-wide 16-byte load reads one contiguous kilobyte;
 *   planes_scales: f16 [T][G][16], the scale of row 16 t + r, group g at [t][g][r];
 *   planes_zeros : u8 [T][G][8], byte j = zero point of row 16 t + 2 j (low nibble), 2 j + 1.
 * Rows past N are zero.  from_planes restores the canonical codes, scales (pad slots 0) and
 * zeros (pad nibbles 0) bit for bit.  codes / planes_codes 16-byte aligned. */
int32_t castforge_hip_int4g_to_planes(const uint32_t *codes, const uint16_t *scales_f16, const uint32_t *zeros,
                                      int64_t rows, int64_t k, int64_t group, void *planes_codes,
                                      uint16_t *planes_scales, uint8_t *planes_zeros, void *stream,
                                      char **out_error);
int32_t castforge_hip_int4g_from_planes(const void *planes_codes, const uint16_t *planes_scales,
                                        const uint8_t *planes_zeros, int64_t rows, int64_t k, int64_t group,
                                        uint32_t *codes, uint16_t *scales_f16, uint32_t *zeros, void *stream,
                                        char **out_error);

/* castforge_hip_gemv_w4a16_batched at M = 1..16 over GEMV planes (codes / scales_f16 / zeros of
 * each problem point at its planes; group 128, k % 128 == 0, x [m, k] and codes 16-byte
 * aligned, y [m, n]): the decode GEMV of `castforge.fused_qmatmul` (codegen/eval.rs:1145-1179,
 * eval_matmul_2d eval.rs:1465-1507) in one launch of one workgroup per CU, every matrix's planes
 * streamed once.  Every finite bf16 x is handled exactly (a power-of-two pre-scale per row and
 * 128 activations, undone on the f32 partial); a non-finite x gives NaN or inf in the rows it
 * reaches.  M = 1: a problem's activations must fit the kernel's LDS (about 2.1 * k bytes; k up
 * to about 65536).  M = 2..16: any k; a workgroup's partials (4 to 8 KB per 16 rows it takes)
 * must fit LDS, which a matrix that would exceed it meets by taking more workgroups. */
int32_t castforge_hip_gemv_w4a16_planes_batched(const cfh_w4a16_problem_t *problems, int32_t count,
                                                int64_t m, int32_t y_dtype, void *stream, char **out_error);

/* The same for INT8 (per-channel or per-tensor scales, k % 64 == 0) and NF4 weights (one block
 * size for the whole batch), e.g. the INT8 block of config 1 or the NF4 MLP of config 3. */
typedef struct cfh_w8a16_problem_t {
    const uint16_t *x;     /* bf16 [M, k] */
    const int8_t *codes;   /* i8 [n, k] */
    const float *scales;   /* f32 [n] (CFH_GRAN_CHANNEL) or [1] (CFH_GRAN_TENSOR) */
    void *y;               /* [M, n] */
    int64_t n, k;
    int32_t granularity;
} cfh_w8a16_problem_t;

int32_t castforge_hip_gemv_w8a16_batched(const cfh_w8a16_problem_t *problems, int32_t count,
                                         int64_t m, int32_t y_dtype, void *stream,
                                         char **out_error);

typedef struct cfh_nf4_problem_t {
    const uint16_t *x;      /* bf16 [M, k] */
    const uint32_t *codes;  /* u32 [n, k/8] */
    const float *absmax;    /* f32 [n, ceil(k/block)] */
    void *y;                /* [M, n] */
    int64_t n, k, block;
} cfh_nf4_problem_t;

int32_t castforge_hip_gemv_nf4_batched(const cfh_nf4_problem_t *problems, int32_t count, int64_t m,
                                       int32_t y_dtype, void *stream, char **out_error);

/* NF4 GEMV planes: the layout of NF4 weights (block a power of two >= 32, K % 128 == 0) that
 * the M = 1 kernel below streams, built once at load time (no reference counterpart: the
 * reference keeps one i8 code per element, ir/tensor_store.rs:44-48).  T = ceil(N/16), G = K/128:
 *   planes_codes : T x G chunks of 1024 bytes; chunk (t, g) holds, at byte 16 * (16 p + r),
 *                  canonical code words 16 g + p, 16 g + 4 + p, 16 g + 8 + p, 16 g + 12 + p of
 *                  row 16 t + r (p = 0..3), so that the q-th words of the four parts are codes
 *                  32 q .. 32 q + 31 of the chunk;
 *   planes_absmax: f32 [T][G][16][nbpc], nbpc = max(1, 128 / block): the absmax of row
 *                  16 t + r for the blocks of chunk g (a block longer than 128 codes repeats its
 *                  absmax in each of its chunks).
 * Rows past N are zero.  from_planes restores the canonical codes u32 [N, K/8] and absmax f32
 * [N, K/block] bit for bit.  planes_codes 16-byte aligned. */
int32_t castforge_hip_nf4_to_planes(const uint32_t *codes, const float *absmax, int64_t rows, int64_t k,
                                    int64_t block, void *planes_codes, float *planes_absmax, void *stream,
                                    char **out_error);
int32_t castforge_hip_nf4_from_planes(const void *planes_codes, const float *planes_absmax, int64_t rows, int64_t k,
                                      int64_t block, uint32_t *codes, float *absmax, void *stream, char **out_error);

/* castforge_hip_gemv_nf4_batched at M = 1 over NF4 planes (codes / absmax of each problem point
 * at its planes; one block size for the batch; x [1, k] and codes 16-byte aligned): the decode
 * GEMV of `castforge.fused_qmatmul` over NF4 weights (codegen/eval.rs:1145-1179, eval_matmul_2d
 * eval.rs:1465-1507, the NF4 dequant of schemes.rs) in one launch of one workgroup per CU.  The
 * weight operands are the exact f16 hi + lo pair of each table value; x is handled as in
 * castforge_hip_gemv_w4a16_planes_batched (power-of-two pre-scale per 128 activations).  A
 * problem's activations must fit LDS next to the 64 KB decode table (k up to about 40000). */
int32_t castforge_hip_gemv_nf4_planes_batched(const cfh_nf4_problem_t *problems, int32_t count, int64_t m,
                                              int32_t y_dtype, void *stream, char **out_error);

/* FP8 E4M3 W8A8 GEMM: y[m, n] = (sum_k e4m3(qa[m,k]) * e4m3(qw[n,k])) * sa[m] * sw[n], stored
 * as bf16 (RNE) or f32 per y_dtype.
 * qa/sa come from castforge_hip_quantize_fp8 on the activations (per token), qw/sw on the
 * weights (per output channel).  New W8A8 path for `castforge.fused_qmatmul` (the reference's
 * fp8 pass, passes/quantize/schemes.rs:633-754, writes dequantized f32 back instead).
 * k % 64 == 0 (k < 2^23) with 16-byte aligned qa/qw runs the fp8 MFMA kernel; other shapes
 * run a one-thread-per-output f32 kernel.
 * Precision: the fp8 MFMA sums each block of eight products in a fixed-point adder aligned to
 * the block's largest product, keeping about 13 bits below it.  On inputs with large outliers
 * a few outputs near zero therefore miss the evaluator's f32 loop (eval.rs:1492-1505) by more
 * than 1e-3 absolute; castforge_hip_gemm_fp8_exact below does not. */
int32_t castforge_hip_gemm_fp8(const uint8_t *qa, const float *sa, int64_t m, const uint8_t *qw,
                               const float *sw, int64_t n, int64_t k, void *y, int32_t y_dtype,
                               void *stream, char **out_error);

/* The same product as castforge_hip_gemm_fp8, with the E4M3 codes widened exactly to f16 and
 * summed on f16 MFMA (exact products, f32-like accumulation): the f32 evaluator's result
 * (eval.rs:1465-1507 on the dequantized operands) within 1e-2 relative / 1e-3 absolute on any
 * input, at about half the fp8 kernel's rate.  Same arguments and shape rules. */
int32_t castforge_hip_gemm_fp8_exact(const uint8_t *qa, const float *sa, int64_t m, const uint8_t *qw,
                                     const float *sw, int64_t n, int64_t k, void *y, int32_t y_dtype,
                                     void *stream, char **out_error);

/* ---- steps either side of the fused matmul ------------------------------------------------- */

/* Epilogue of `castforge.fused_qmatmul` (codegen/eval.rs:1151-1176), in place on f32 y[count]:
 * val = y[i] + bias[i % bias_len]; RELU: max(val, z[i % z_len]); TANH: tanh(val); SILU:
 * val / (1 + exp(-val)); GELU: the tanh form of eval.rs:1733-1735; SCALE: val * z[i % z_len];
 * BIAS: val.  z_len == 0 means z = 0 (the evaluator's default). */
enum { CFH_EPI_BIAS = 0, CFH_EPI_RELU = 1, CFH_EPI_TANH = 2, CFH_EPI_SILU = 3, CFH_EPI_GELU = 4,
       CFH_EPI_SCALE = 5 };
int32_t castforge_hip_qmatmul_epilogue(float *y, int64_t count, const float *bias, int64_t bias_len,
                                       const float *z, int64_t z_len, int32_t kind, void *stream,
                                       char **out_error);

/* f32 -> bf16 with round-to-nearest-even (NaN stays NaN): the bf16 activations the fused
 * matmul consumes after `lower-mixed-precision` (passes/quantize/formats.rs:563-591).  The
 * reference's evaluator treats that convert as a copy (codegen/eval.rs:674-676); here the
 * operand really is bf16. */
int32_t castforge_hip_convert_f32_to_bf16(const float *src, int64_t n, uint16_t *dst, void *stream,
                                          char **out_error);
int32_t castforge_hip_convert_bf16_to_f32(const uint16_t *src, int64_t n, float *dst, void *stream,
                                          char **out_error);

/* y[i] = clamp(round_half_away(x[i] / scale), -qmax, qmax) * scale in f32, qmax = 7 for bits == 4
 * and 127 otherwise, NaN kept: the `castforge.static_quantize` op that calibrate-quantize
 * (quantize(scheme=w8a8), passes/quantize/formats.rs:15-113) inserts before each matmul's
 * activations, evaluated as codegen/eval.rs:1369-1382 does.  scale is the attribute already
 * resolved to f32 (> 0). */
int32_t castforge_hip_static_quantize(const float *x, int64_t n, float scale, int32_t bits, float *y,
                                      void *stream, char **out_error);

/* ---- outlier suppression (passes/quantize/formats.rs:230-343, schemes.rs:155-298) ------------ */

/* Replaces RotateHadamardPass::run's loop (formats.rs:303-327): dst = the Walsh-Hadamard
 * rotation of f32 [d0, d1] in blocks of `block` consecutive elements along `axis`: each block
 * through the radix-2 butterfly (x + y, x - y; stages h = 1, 2, .., block/2 in order), then
 * times 1.0f / sqrtf(block).  axis 0 rotates down the columns as the reference does for a
 * [k, n] constant; axis 1 along rows (the K axis of an [N, K] weight or of activations).
 * block: a power of two >= 2 dividing the axis length (the pass resolves the reference's
 * next_power_of_two(block_size).min(k).max(2) and skips the rotation when k % b != 0).
 * dst may equal src.  Bit-exact with the reference's f32 loop. */
int32_t castforge_hip_rotate_hadamard(const float *src, int64_t d0, int64_t d1, int64_t block, int32_t axis,
                                      float *dst, void *stream, char **out_error);

/* INT4g quantization of the row-wise Hadamard rotation of src [rows, cols] in one pass: the
 * codes castforge_hip_quantize_int4g gives for castforge_hip_rotate_hadamard(src, rows, cols,
 * block, axis 1), without writing the rotated f32 tensor.  This is the K-axis rotation of
 * QuaRot on an [N, K] weight, equal to rotate-hadamard on the [K, N] form followed by
 * pack-weights.  group: power of two in [16, 256]; block: power of two in [2, 1024]
 * dividing cols. */
int32_t castforge_hip_quantize_int4g_hadamard(const float *src, int64_t rows, int64_t cols, int64_t group,
                                              int64_t block, uint32_t *codes, uint16_t *scales_f16,
                                              uint32_t *zeros, void *stream, char **out_error);

/* SmoothQuant scalars of schemes.rs:231-233 (host arithmetic, no device work), with act_max
 * the constant's calibrated bound, w_max = max(max |w|, 1e-5) and alpha already clamped to
 * [0.05, 0.95]: out_scales[0] = s = max(max(act_max, 1e-4)^alpha / w_max^(1 - alpha), 1e-4),
 * out_scales[1] = e = max(w_max * s / qmax, 1e-6), qmax = 7 (bits 4) or 127; powf is the C
 * library's, as f32::powf is in the reference. */
int32_t castforge_hip_smoothquant_scales(float act_max, float w_max, float alpha, int32_t bits, float *out_scales,
                                         char **out_error);
/* Replaces the element loop of run_smoothquant (schemes.rs:234-238): out[i] =
 * (clamp(round_half_away((w[i] * s) / e), qmin, qmax) * e) / s, NaN kept, [qmin, qmax] =
 * [-8, 7] (bits 4) or [-128, 127].  out may equal w. */
int32_t castforge_hip_smoothquant(const float *w, int64_t n, float smooth_scale, float eff_qscale, int32_t bits,
                                  float *out, void *stream, char **out_error);

/* ---- GGUF payloads (ir/formats/gguf.rs) --------------------------------------------------- */

/* GgmlType ids of the reference's GGUF reader / writer (gguf.rs:16-37). */
enum { CFH_GGML_F32 = 0, CFH_GGML_F16 = 1, CFH_GGML_Q4_0 = 2, CFH_GGML_Q8_0 = 8, CFH_GGML_BF16 = 30 };

/* One matrix of castforge_hip_gemv_gguf_batched: x bf16 [m, k], GGUF planes of W [n, k], y [m, n]. */
typedef struct {
    const uint16_t *x;
    const void *codes;
    const uint16_t *scales_f16;
    void *y;
    int64_t n, k;
} cfh_gguf_problem_t;

/* Payload bytes of num_elems elements (gguf.rs:491-550: F32 4 B, F16 / BF16 2 B, Q4_0 18 B and
 * Q8_0 34 B per started block of 32).  Unknown ids fail with the reference's message. */
int32_t castforge_hip_gguf_payload_bytes(int32_t ggml_type, int64_t num_elems, int64_t *out_bytes,
                                         char **out_error);

/* Replaces decode_ggml_tensor (gguf.rs:486-550): num_elems f32 values of a tensor payload.
 * Q4_0: blocks of f16 d + 16 bytes, element 2j = low nibble of byte j, 2j+1 = high nibble,
 * value (nibble - 8) * d; Q8_0: f16 d + 32 int8, value q * d; F16 exactly as
 * f16_bits_to_f32 (ir/tensor_store.rs:59-82); BF16 as bits << 16.  Blocks run over the
 * flattened tensor and the last one may be partial.  raw: device, 4-byte (F32) or 2-byte
 * aligned, holding payload_bytes(type, num_elems) bytes. */
int32_t castforge_hip_gguf_decode(int32_t ggml_type, const void *raw, int64_t num_elems, float *out,
                                  void *stream, char **out_error);

/* Replaces the payload loop of export_gguf_bytes (gguf.rs:280-322).  Q8_0: src = int8 codes of a
 * QuantizedI8 tensor and `scale` its one scale, written into every block as
 * f32_to_f16_bits(scale) (truncating, tensor_store.rs:84-102), codes past num_elems 0, and
 * ceil(max(num_elems, 1) / 32) blocks (gguf.rs:283-296).  F16 / BF16: src = f32 values, by the
 * truncating converters (tensor_store.rs:84-111).  F32: a copy.  scale is ignored but for Q8_0. */
int32_t castforge_hip_gguf_encode(int32_t ggml_type, const void *src, int64_t num_elems, float scale,
                                  void *raw_out, void *stream, char **out_error);

/* GGUF planes: the layout castforge_hip_gemv_gguf reads, for a Q4_0 / Q8_0 matrix [rows, k] whose
 * blocks run along k (row-major after the reader's dimension reversal, gguf.rs:117-122).
 * codes: rows x (k/2) bytes (Q4_0) or rows x k (Q8_0); each row is cut into chunks of 128
 * (Q4_0) / 64 (Q8_0) elements = 64 bytes, stored as four 16-byte parts, part p holding
 * elements 8p..8p+7 of each block of the chunk (Q4_0: 4 bytes per block in the block's nibble
 * order; Q8_0: 8 bytes per block).  scales_f16: the blocks' d bits [rows, GP],
 * GP = 8 * ceil(k/32 / 8), pad slots 0.  Needs k % 128 == 0 (Q4_0) or k % 64 == 0 (Q8_0) and
 * 16-byte aligned planes.  No reference counterpart: the reference decodes to f32 on import. */
int32_t castforge_hip_gguf_repack(int32_t ggml_type, const void *raw, int64_t rows, int64_t k, void *codes,
                                  uint16_t *scales_f16, void *stream, char **out_error);
/* Planes back to the block payload (the inverse of castforge_hip_gguf_repack). */
int32_t castforge_hip_gguf_unpack(int32_t ggml_type, const void *codes, const uint16_t *scales_f16, int64_t rows,
                                  int64_t k, void *raw_out, void *stream, char **out_error);
/* Q4_0 planes to the INT4g layout (group 32, every zero point 8): int4_codes u32 [rows, k/8],
 * zeros u32 [rows, ceil(k/32 / 8)] = 0x88888888; the planes' scales_f16 serve unchanged as
 * INT4g scales.  (q - 8) * d is the INT4g dequant of the same block, so castforge_hip_gemv_w4a16
 * (prefill MFMA kernel at M > 64) then computes the Q4_0 matmul. */
int32_t castforge_hip_gguf_q4_0_to_int4g(const void *codes, int64_t rows, int64_t k, uint32_t *int4_codes,
                                         uint32_t *zeros, void *stream, char **out_error);
/* Planes to f32 [rows, k]: the values decode_ggml_tensor gives for the same blocks. */
int32_t castforge_hip_dequantize_gguf(int32_t ggml_type, const void *codes, const uint16_t *scales_f16,
                                      int64_t rows, int64_t k, float *out, void *stream, char **out_error);

/* y[m, n] = sum_k x[m, k] * decode(W)[n, k] over GGUF planes of a Q4_0 / Q8_0 matrix W [n, k]
 * (contraction along the blocked dimension, as GGUF producers store linear weights).  The
 * dequant-GEMV of a GGUF weight: the reference decodes it to f32 (gguf.rs:513-550) and
 * evaluates the matmul (codegen/eval.rs:1465-1507).  x bf16 [m, k] 16-byte aligned; y f32 or
 * bf16.  M = 1 and 2 run the split-K MFMA kernel (one MFMA per block, scaled in f32 by its d;
 * M = 2 as two problems of one launch), M = 3..64 (Q4_0: 3..32) the skinny MFMA kernel (the
 * same per-block MFMA, x read per wave); larger M the prefill MFMA kernel
 * reading the planes directly (exact hi / lo f16 planes of the block values, which must lie
 * within f16 range); shapes neither fits take a generic kernel. */
int32_t castforge_hip_gemv_gguf(int32_t ggml_type, const uint16_t *x, int64_t m, int64_t n, int64_t k,
                                const void *codes, const uint16_t *scales_f16, void *y, int32_t y_dtype,
                                void *stream, char **out_error);
/* Up to CFH_MAX_BATCH matrices of one type with the same M (1..64) in one launch. */
int32_t castforge_hip_gemv_gguf_batched(int32_t ggml_type, const cfh_gguf_problem_t *problems, int32_t count,
                                        int64_t m, int32_t y_dtype, void *stream, char **out_error);

/* Q4_0 GEMV planes: GGUF Q4_0 planes (castforge_hip_gguf_repack) of a [rows, k] matrix
 * (k % 128 == 0) rewritten once, at load, for the M = 1 decode kernel below (no reference
 * counterpart).  T = ceil(rows/16), G = k/128:
 *   planes_codes: T x G chunks of 1024 bytes; chunk (t, g) holds, at byte 16 * (16 p + r), the
 *                 16-byte part p of chunk g of row 16 t + r of the GGUF planes (elements
 *                 8p..8p+7 of its four blocks);
 *   planes_d    : f16 [T][G][16][4], the d of blocks 4g..4g+3 of row 16 t + r.
 * Rows past `rows` are zero.  from_gemv_planes restores the GGUF planes (pad d slots 0) bit for
 * bit.  codes and planes_codes 16-byte aligned, planes_d 8-byte aligned. */
int32_t castforge_hip_gguf_q4_0_to_gemv_planes(const void *codes, const uint16_t *scales_f16, int64_t rows, int64_t k,
                                              void *planes_codes, uint16_t *planes_d, void *stream, char **out_error);
int32_t castforge_hip_gguf_q4_0_from_gemv_planes(const void *planes_codes, const uint16_t *planes_d, int64_t rows,
                                                int64_t k, void *codes, uint16_t *scales_f16, void *stream,
                                                char **out_error);
/* castforge_hip_gemv_gguf_batched for Q4_0 at M = 1 over Q4_0 GEMV planes (codes / scales_f16
 * of each problem point at its planes; x [1, k] 16-byte aligned): y = x * decode(W)^T as the
 * reference decodes Q4_0 (gguf.rs:513-550) and evaluates the matmul (codegen/eval.rs:1465-1507),
 * in one launch of one workgroup per CU.  Each block's products are exact ((q - 8) in f16, x
 * with a power-of-two pre-scale per 128 activations) and its f32 sum is scaled by its d. */
int32_t castforge_hip_gemv_gguf_q4_0_planes_batched(const cfh_gguf_problem_t *problems, int32_t count, int64_t m,
                                                   int32_t y_dtype, void *stream, char **out_error);

/* *out = max |src[i]| over the non-NaN elements (0 for n == 0), written on the device: the
 * constant ranges of calibrate-quantize's calibrate_value_ranges (formats.rs:135-150). */
int32_t castforge_hip_absmax_f32(const float *src, int64_t n, float *out, void *stream, char **out_error);

/* dst[c, r] = src[r, c] for [rows, cols] elements of elem_bytes (1, 2 or 4): the [K, N] ->
 * [N, K] transpose of PackWeightsPass (passes/weights/fold.rs:549-554). */
int32_t castforge_hip_transpose(const void *src, int64_t rows, int64_t cols, int32_t elem_bytes, void *dst,
                                void *stream, char **out_error);

/* out[m, n] = sum_k a[m, k] * b[k, n] (or b[n, k] when packed_rhs), f32 operands, k ascending
 * with separate multiply and add per output: bit-identical to eval_matmul_2d
 * (codegen/eval.rs:1465-1507).  The evaluator's unfused dot_general; the quantized hot path
 * is castforge_hip_gemv_* / castforge_hip_gemm_fp8. */
int32_t castforge_hip_matmul_f32(const float *a, int64_t m, int64_t k, const float *b, int64_t n,
                                 int32_t packed_rhs, float *out, void *stream, char **out_error);

#ifdef __cplusplus
}
#endif

#endif /* CASTFORGE_HIP_H */
