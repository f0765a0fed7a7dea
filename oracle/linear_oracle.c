/*
 * CPU oracle for the Linear hot path — TEST INFRASTRUCTURE ONLY (see
 * linear_oracle.h for what it restates and how each function is pinned).
 *
 * Built with -ffp-contract=off so that every fused multiply-add is an
 * explicit fmaf() where the reference writes one, and every other product
 * and sum rounds separately, as the reference's host code does.
 */
#include "linear_oracle.h"

#include <math.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

int orc_default_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

static int resolve_threads(int threads) {
  return threads > 0 ? threads : orc_default_threads();
}

/* export_model.py:123-131: bits + 0x7FFF + ((bits >> 16) & 1), then >> 16;
 * a NaN keeps its high half with the quiet bit 0x0040 set. */
uint16_t orc_f32_to_bf16(float value) {
  uint32_t bits;
  memcpy(&bits, &value, sizeof bits);
  if ((bits & 0x7F800000u) == 0x7F800000u && (bits & 0x007FFFFFu) != 0u) {
    return (uint16_t)((bits >> 16) | 0x0040u);
  }
  bits += 0x7FFFu + ((bits >> 16) & 1u);
  return (uint16_t)(bits >> 16);
}

/* export_model.py:134-136: the BF16 word is the high half of the float. */
float orc_bf16_to_f32(uint16_t value) {
  const uint32_t bits = (uint32_t)value << 16;
  float result;
  memcpy(&result, &bits, sizeof result);
  return result;
}

void orc_f32_to_bf16_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(in[i]);
}

void orc_bf16_to_f32_array(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(in[i]);
}

/* A fixed, blocked FP32 dot product: eight running FMA lanes over k in steps
 * of eight, folded pairwise, then the tail in order.  This stands in for
 * OpenBLAS's sgemv kernel, whose order is unspecified (and unpinned). */
static float dot_blocked(const float* a, const float* b, int n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int k = 0;
  for (; k + 8 <= n; k += 8) {
    for (int j = 0; j < 8; ++j) acc[j] = fmaf(a[k + j], b[k + j], acc[j]);
  }
  float sum = ((acc[0] + acc[4]) + (acc[1] + acc[5])) +
              ((acc[2] + acc[6]) + (acc[3] + acc[7]));
  for (; k < n; ++k) sum = fmaf(a[k], b[k], sum);
  return sum;
}

/* cpu_ops.cpp:23-30. */
void orc_linear_fp32(const float* weight, const float* bias, const float* input,
                     float* output, int out_features, int in_features,
                     int threads) {
  const int nt = resolve_threads(threads);
#pragma omp parallel for num_threads(nt) schedule(static)
  for (int row = 0; row < out_features; ++row) {
    output[row] =
        dot_blocked(weight + (size_t)row * in_features, input, in_features);
  }
  if (bias) {
    for (int row = 0; row < out_features; ++row) output[row] += bias[row];
  }
}

/* cpu_ops.cpp:108-123.  Rows of W outer so that each weight row is reused
 * from cache across all tokens. */
void orc_linear_fp32_batch(const float* weight, const float* bias,
                           const float* input, float* output, int token_count,
                           int out_features, int in_features, int threads) {
  const int nt = resolve_threads(threads);
#pragma omp parallel for num_threads(nt) schedule(static)
  for (int row = 0; row < out_features; ++row) {
    const float* w = weight + (size_t)row * in_features;
    for (int token = 0; token < token_count; ++token) {
      output[(size_t)token * out_features + row] = dot_blocked(
          w, input + (size_t)token * in_features, in_features);
    }
  }
  if (bias) {
    for (int token = 0; token < token_count; ++token) {
      float* out_row = output + (size_t)token * out_features;
      for (int row = 0; row < out_features; ++row) out_row[row] += bias[row];
    }
  }
}

/* cpu_ops.cpp:175-177: std::max_element returns the first maximum. */
int orc_argmax(const float* values, int n) {
  if (n <= 0) return -1;
  int best = 0;
  for (int i = 1; i < n; ++i) {
    if (values[i] > values[best]) best = i;
  }
  return best;
}

int orc_dequant_w8a16(const int8_t* weight, const uint16_t* scales,
                      int group_size, int out_features, int in_features,
                      float* output, int threads) {
  if (group_size <= 0) return -1;
  const int groups = (in_features + group_size - 1) / group_size;
  const int nt = resolve_threads(threads);
#pragma omp parallel for num_threads(nt) schedule(static)
  for (int row = 0; row < out_features; ++row) {
    const int8_t* q = weight + (size_t)row * in_features;
    const uint16_t* s = scales + (size_t)row * groups;
    float* w = output + (size_t)row * in_features;
    for (int k = 0; k < in_features; ++k) {
      w[k] = (float)q[k] * orc_bf16_to_f32(s[k / group_size]);
    }
  }
  return 0;
}

/* test_cuda.cpp:492-517. */
int orc_w8a16_reference(const int8_t* weight, const uint16_t* scales,
                        int group_size, const uint16_t* bias,
                        const uint16_t* input, float* output_f32,
                        uint16_t* output_bf16, int token_count,
                        int out_features, int in_features, int threads) {
  if (group_size <= 0) return -1;
  const int groups = (in_features + group_size - 1) / group_size;
  const int nt = resolve_threads(threads);
#pragma omp parallel for num_threads(nt) schedule(static)
  for (int row = 0; row < out_features; ++row) {
    const int8_t* q = weight + (size_t)row * in_features;
    const uint16_t* s = scales + (size_t)row * groups;
    for (int token = 0; token < token_count; ++token) {
      const uint16_t* x = input + (size_t)token * in_features;
      float sum = 0.0f;
      for (int k = 0; k < in_features; ++k) {
        const float dequantized =
            (float)q[k] * orc_bf16_to_f32(s[k / group_size]);
        sum = fmaf(dequantized, orc_bf16_to_f32(x[k]), sum);
      }
      if (bias) sum += orc_bf16_to_f32(bias[row]);
      const size_t at = (size_t)token * out_features + row;
      if (output_f32) output_f32[at] = sum;
      if (output_bf16) output_bf16[at] = orc_f32_to_bf16(sum);
    }
  }
  return 0;
}

/* test_cuda.cpp:474-490. */
void orc_bf16_linear_reference(const uint16_t* weight, const uint16_t* bias,
                               const uint16_t* input, float* output,
                               int token_count, int out_features,
                               int in_features, int threads) {
  const int nt = resolve_threads(threads);
#pragma omp parallel for num_threads(nt) schedule(static)
  for (int row = 0; row < out_features; ++row) {
    const uint16_t* w = weight + (size_t)row * in_features;
    for (int token = 0; token < token_count; ++token) {
      const uint16_t* x = input + (size_t)token * in_features;
      float sum = bias ? orc_bf16_to_f32(bias[row]) : 0.0f;
      for (int k = 0; k < in_features; ++k) {
        const float product = orc_bf16_to_f32(w[k]) * orc_bf16_to_f32(x[k]);
        sum = sum + product;
      }
      output[(size_t)token * out_features + row] = sum;
    }
  }
}

/* qwen2.cpp:421-424 on the CPU branch: linear(lm_head) then argmax. */
int orc_lm_head(const uint16_t* weight, const uint16_t* input, int vocab,
                int in_features, float* logits_f32, uint16_t* logits_bf16,
                int threads) {
  const int nt = resolve_threads(threads);
  float h[8192];
  if (in_features <= 0 || in_features > 8192) return -1;
  orc_bf16_to_f32_array(input, h, (size_t)in_features);
#pragma omp parallel num_threads(nt)
  {
    float row_f32[8192];
#pragma omp for schedule(static)
    for (int row = 0; row < vocab; ++row) {
      orc_bf16_to_f32_array(weight + (size_t)row * in_features, row_f32,
                            (size_t)in_features);
      logits_f32[row] = dot_blocked(row_f32, h, in_features);
    }
  }
  if (logits_bf16) {
    for (int row = 0; row < vocab; ++row) {
      logits_bf16[row] = orc_f32_to_bf16(logits_f32[row]);
    }
  }
  return orc_argmax(logits_f32, vocab);
}
