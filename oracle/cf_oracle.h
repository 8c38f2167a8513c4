/*
 * CPU oracle for the quantized-weight hot path — TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker that GPU results are compared against.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The product
 * (castforge_amd, libcastforge_hip.so) never links, loads or falls back to it.
 *
 * Two kinds of functions live here:
 *   - restatements of the reference's CPU algorithms (file:line of sungdomo/CastForge
 *     cited on each function), pinned by the reference's own known-answer tests;
 *   - the written spec of the schemes that the reference does not implement
 *     (per-channel INT8, INT4 asymmetric group-wise packed, NF4 block-wise, FP8 E4M3
 *     per-row W8A8).  Those are "parity unpinned" by the reference and are pinned by
 *     closed forms, independent restatements and brute force in tests/.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math) -> oracle/_build/.
 */
#ifndef CF_ORACLE_H
#define CF_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_ROUND_HALF_AWAY = 0, ORC_ROUND_HALF_EVEN = 1 };

/* ---- scalar converters ---------------------------------------------------------------- */
/* tensor_store.rs:59-111 (reference, truncating) */
uint16_t orc_f32_to_bf16_trunc(float v);
uint16_t orc_f32_to_f16_trunc(float v);
float orc_f16_to_f32(uint16_t h);
float orc_bf16_to_f32(uint16_t b);
/* IEEE round-to-nearest-even converters used by the new packed formats */
uint16_t orc_f32_to_bf16_rne(float v);
uint16_t orc_f32_to_f16_rne(float v);

/* mutable_loads.rs:367-441 — OCP E4M3FN codec (faithful restatement) */
uint8_t orc_f32_to_e4m3fn(float v);
float orc_e4m3fn_to_f32(uint8_t b);
/* independent integer RNE + saturate-to-finite encoder (used to pin the codec) */
uint8_t orc_f32_to_e4m3fn_int(float v);
/* integer encoder plus the reference's 16-input log2 quirk: must equal orc_f32_to_e4m3fn on
 * every f32 (this is the rule the GPU encoder implements) */
uint8_t orc_f32_to_e4m3fn_fast(float v);
/* compare the faithful codec with the integer encoder (use_fast=0) or with the quirk-aware
 * encoder (use_fast=1) over the f32 bit patterns [lo, hi) with the given stride; returns the
 * number of mismatches and writes the smallest mismatching pattern to *first_bad */
int64_t orc_e4m3_crosscheck(uint32_t lo, uint32_t hi, uint32_t stride, int use_fast,
                            uint32_t *first_bad);

/* ---- reference quantizers -------------------------------------------------------------- */
/* formats.rs:654-660 */
void orc_int_bounds(int bits, int *eff_bits, float *qmin, float *qmax);
/* formats.rs:664-678: per-tensor symmetric; returns scale */
float orc_quantize_symmetric(const float *v, int64_t n, int bits, int round_mode, int8_t *q);
/* formats.rs:680-688: scale string "{:.6}" with trailing zeros trimmed */
void orc_scale_string(float scale, char *buf, int buflen);
/* schemes.rs:485-549: group-wise / AWQ symmetric dequantize-in-place over the flattened
 * tensor; returns the salient count; writes dequantized values and per-group scales */
int64_t orc_quantize_groupwise(const float *v, int64_t n, int bits, int64_t group_size,
                               int awq_salient, float salient_ratio, int round_mode,
                               float *deq, float *scales, float *salient_thresh);
/* schemes.rs:681-713: FP8 / MXFP8 uniform-grid dequantize-in-place */
void orc_quantize_fp8_grid(const float *v, int64_t n, int e5m2, int mxfp8, int64_t block_size,
                           float *deq);

/* ---- BASELINE schemes (written spec; parity unpinned by the reference) ----------------- */
/* INT8/INT4 symmetric per output channel: rows of [n, k], one scale per row */
void orc_quantize_int8_rows(const float *v, int64_t n, int64_t k, int bits, int round_mode,
                            int8_t *q, float *scales);
/* INT4 asymmetric group-wise along K with fp16 scale and u4 zero-point, 8 codes / u32;
 * scales are [n][8*ceil(G/8)] (row-padded, pad 0), zeros [n][ceil(G/8)] */
void orc_quantize_int4g(const float *v, int64_t n, int64_t k, int64_t group, uint32_t *codes,
                        uint16_t *scales_f16, uint32_t *zeros);
void orc_dequantize_int4g(const uint32_t *codes, const uint16_t *scales_f16,
                          const uint32_t *zeros, int64_t n, int64_t k, int64_t group, float *out);
/* NF4 block-wise absmax along K, 8 codes / u32 */
extern const float ORC_NF4_TABLE[16];
uint8_t orc_nf4_code(float x);
void orc_quantize_nf4(const float *v, int64_t n, int64_t k, int64_t block, uint32_t *codes,
                      float *absmax);
void orc_dequantize_nf4(const uint32_t *codes, const float *absmax, int64_t n, int64_t k,
                        int64_t block, float *out);
/* FP8 E4M3 per-row (weights) / per-token (activations) absmax/448 scale */
void orc_quantize_fp8_rows(const float *v, int64_t rows, int64_t cols, uint8_t *codes,
                           float *scales);
void orc_quantize_fp8_rows_bf16(const uint16_t *v, int64_t rows, int64_t cols, uint8_t *codes,
                                float *scales);

/* ---- evaluator GEMM semantics ---------------------------------------------------------- */
/* eval.rs:1465-1507: out[m,n] = sum_k a[m,k]*b[...]; f32 acc, separate mul/add, k ascending */
void orc_matmul_2d(const float *a, const float *b, int64_t m, int64_t n, int64_t k,
                   int packed_rhs, float *out);
/* eval.rs:1151-1176: fused_qmatmul epilogues; mode 0 none 1 bias 2 bias_relu 3 bias_tanh
 * 4 bias_silu 5 bias_gelu 6 bias_scale */
void orc_epilogue(float *out, int64_t len, const float *bias, int64_t bias_len, const float *z,
                  int64_t z_len, int mode);
/* dequant-then-matmul oracles for the packed formats; x is bf16 [m,k], out f32 [m,n] */
void orc_gemm_w8a16(const uint16_t *x, int64_t m, int64_t n, int64_t k, const int8_t *codes,
                    const float *scales, float *out);
void orc_gemm_w4a16(const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t group,
                    const uint32_t *codes, const uint16_t *scales_f16, const uint32_t *zeros,
                    float *out);
void orc_gemm_nf4(const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t block,
                  const uint32_t *codes, const float *absmax, float *out);
/* codegen/eval.rs:1369-1382: castforge.static_quantize (fake quant of a matmul's activations) */
void orc_static_quantize(const float *x, int64_t n, float sc, int bits, float *y);

/* gguf.rs:16-23 (GgmlType ids) and gguf.rs:486-550 / 283-296 (payload decode, Q8_0 encode) */
enum { ORC_GGML_F32 = 0, ORC_GGML_F16 = 1, ORC_GGML_Q4_0 = 2, ORC_GGML_Q8_0 = 8, ORC_GGML_BF16 = 30 };
int64_t orc_gguf_decode(int type, const uint8_t *raw, int64_t num_elems, float *out);
int64_t orc_gguf_encode_q8_0(const int8_t *codes, int64_t n, float scale, uint8_t *out);

/* formats.rs:301-327 (rotate-hadamard of a [k, n] constant, in place; returns b or -1) and
 * schemes.rs:188-238 (smooth-quantize of one constant, in place) */
int64_t orc_rotate_hadamard(float *w, int64_t k, int64_t n, int64_t block_size);
void orc_smoothquant(float *w, int64_t n, float act_max, float alpha, int bits, float *scales_out);

void orc_gemm_fp8(const uint8_t *qa, const float *sa, int64_t m, const uint8_t *qw,
                  const float *sw, int64_t n, int64_t k, float *out);

/* timing helper for the CPU baseline: quantize_int4g + gemv over a row slice */
double orc_now_seconds(void);

void orc_quantize_int4g_awq(const float *v, const float *s, int64_t n, int64_t k, int64_t group,
                            uint32_t *codes, uint16_t *scales_f16, uint32_t *zeros);
/* closed form of the MX scale exponent ceilf(log2f(raw)) (schemes.rs:706) and its check */
int orc_mx_scale_exp_model(float raw);
int64_t orc_mx_scale_crosscheck(uint32_t lo, uint32_t hi, uint32_t *first_bad);

#ifdef __cplusplus
}
#endif
#endif
