/*
 * CPU oracle for the Linear hot path — TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference engine's CPU FP32 path
 * (src/cpu_ops.cpp, include/infer/cpu_ops.hpp) plus the host-side reference
 * closed forms its tests use (tests/test_cuda.cpp:474-517, 16-29) and the
 * BF16 conversion of the exporter (tools/export_model.py:123-136).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker or the timed CPU baseline.
 * The product path (the HIP library) never calls it.
 *
 * Pinning (what checks each function against something other than itself):
 *   orc_f32_to_bf16 / orc_bf16_to_f32  known answers of the reference's own
 *       self-test (export_model.py:414-428) and test_core.cpp:53,117-118,
 *       plus an exhaustive comparison with numpy's independent bit method.
 *   orc_linear_fp32 / orc_linear_fp32_batch  float64 brute force and
 *       numpy/BLAS matmul on random inputs; batch == per-row (test_ops.cpp:
 *       133-163); linearity in x; identity / permutation weights.
 *   orc_dequant_w8a16  bitwise against float64 q*s (the product is exact in
 *       FP32, at most 16 significant bits); zero-group and +-127 fixtures.
 *   orc_w8a16_reference  golden vectors of the reference's generator
 *       (test_cuda.cpp:519-609) computed in float64 by tests/golden.
 *   orc_argmax  first-max semantics: planted ties (test_cuda.cpp:790-880).
 * OpenBLAS's summation order is not pinned (not vendored, no golden values);
 * every function here is checked to a stated tolerance, not to its order.
 */
#ifndef LINEAR_ORACLE_H
#define LINEAR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* BF16 round-to-nearest-even with NaN quieted (export_model.py:123-131). */
uint16_t orc_f32_to_bf16(float value);
/* BF16 -> FP32 widening (export_model.py:134-136). */
float orc_bf16_to_f32(uint16_t value);
void orc_f32_to_bf16_array(const float* in, uint16_t* out, size_t n);
void orc_bf16_to_f32_array(const uint16_t* in, float* out, size_t n);

/* y = W x (+ bias), W row-major [n_out, n_in]: cpu_ops.cpp:23-30
 * (cblas_sgemv RowMajor NoTrans, then the bias loop). */
void orc_linear_fp32(const float* weight, const float* bias, const float* input,
                     float* output, int out_features, int in_features,
                     int threads);

/* Y = X W^T (+ bias) for token_count rows: cpu_ops.cpp:108-123
 * (cblas_sgemm RowMajor NoTrans x Trans, then the bias loop). */
void orc_linear_fp32_batch(const float* weight, const float* bias,
                           const float* input, float* output, int token_count,
                           int out_features, int in_features, int threads);

/* First index of the maximum: cpu_ops.cpp:175-177 (std::max_element). */
int orc_argmax(const float* values, int n);

/* Exact dequantization w[n,k] = q[n,k] * s[n, k / group] in FP32, with the
 * scale row stride ceil(K / group) (export_model.py:228-242;
 * test_cuda.cpp:499-505; linear_benchmark.cpp:202-207).  Returns 0, or -1
 * when group_size <= 0. */
int orc_dequant_w8a16(const int8_t* weight, const uint16_t* scales,
                      int group_size, int out_features, int in_features,
                      float* output, int threads);

/* The reference's host W8A16 closed form (test_cuda.cpp:492-517): for each
 * output, a sequential FMA chain of fl32(q*s) * x over k, then + bias, then
 * BF16 RNE.  output_f32 (may be NULL) receives the sum before rounding. */
int orc_w8a16_reference(const int8_t* weight, const uint16_t* scales,
                        int group_size, const uint16_t* bias,
                        const uint16_t* input, float* output_f32,
                        uint16_t* output_bf16, int token_count,
                        int out_features, int in_features, int threads);

/* The reference's host BF16 linear closed form (test_cuda.cpp:474-490):
 * sum starts at bias, then += w*x in k order, FP32, on BF16-decoded
 * operands.  Output is FP32 (the test compares against it unrounded). */
void orc_bf16_linear_reference(const uint16_t* weight, const uint16_t* bias,
                               const uint16_t* input, float* output,
                               int token_count, int out_features,
                               int in_features, int threads);

/* The CPU FP32 LM head step (qwen2.cpp:421-424): logits = E h in FP32 on
 * BF16-decoded E and h (rows decoded on the fly, same blocked dot as
 * orc_linear_fp32), then orc_argmax.  logits_f32 must hold vocab floats;
 * logits_bf16 may be NULL.  Returns the argmax index. */
int orc_lm_head(const uint16_t* weight, const uint16_t* input, int vocab,
                int in_features, float* logits_f32, uint16_t* logits_bf16,
                int threads);

/* Number of OpenMP threads a call with threads <= 0 uses. */
int orc_default_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* LINEAR_ORACLE_H */
