/*
 * CPU oracle for the decode step around the Linear path — TEST
 * INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference engine's CPU FP32 model path: the
 * non-Linear ops of src/cpu_ops.cpp (rms_norm 15-21, rope 33-56,
 * attention_decode 58-91, silu_mul 168-173, embedding / store_kv /
 * attention_prefill 93-166) and the op order of Qwen2Model's CPU decode
 * (src/qwen2.cpp:376-425) and matrixized prefill (427-494), on FP32 weights
 * (the W8A16 model's weights dequantised exactly, q * s).  Linear layers use
 * orc_linear_fp32 / orc_linear_fp32_batch of linear_oracle.c.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, as the checker or the timed CPU baseline; the product
 * (the HIP library) never calls it.
 *
 * Pinning (checked against something other than the formula restated here):
 *   orc_rms_norm   the closed form of test_ops.cpp:124-131 (constant input
 *                  c: output = c / sqrt(c^2 + eps) * w) and float64 brute
 *                  force;
 *   orc_rope       position 0 is the identity (test_ops.cpp:166-174); the
 *                  rotation preserves each pair's norm; float64 brute force
 *                  of the rotate-half formula; q and k heads independent;
 *   orc_attention_decode  one position returns that position's value row;
 *                  equal keys give the mean of the values; float64 softmax
 *                  brute force; GQA head -> kv head mapping by a planted
 *                  value per kv head;
 *   orc_silu_mul   float64 closed form and the SiLU fixed points
 *                  (silu(0) = 0, silu(x) -> x for large x);
 *   orc_model_*    prefill of n tokens == n decode steps (the reference's
 *                  test_qwen2.cpp:450-488 checks its CPU paths the same way)
 *                  and a float64 re-implementation of one layer on tiny
 *                  shapes (tests/test_model_oracle.py).
 * The transcendental functions (powf, cosf, sinf, expf, sqrtf) are the C
 * library's; the reference calls the C++ <cmath> overloads of the same
 * functions, whose last-bit results are not pinned here (tolerances only).
 */
#ifndef MODEL_ORACLE_H
#define MODEL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* cpu_ops.cpp:15-21: double sum of squares, scale = 1 / sqrt(sum / n + eps)
 * in float, output = input * scale * weight. */
void orc_rms_norm(const float* input, const float* weight, float* output, int n,
                  float epsilon);

/* cpu_ops.cpp:33-56: rotate-half RoPE of every q and k head at `position`,
 * frequency = theta^(-2 i / head_dim) (powf), angle = position * frequency. */
void orc_rope(float* q, float* k, int num_heads, int num_kv_heads, int head_dim,
              int position, float theta);

/* cpu_ops.cpp:58-91: softmax(q K^T / sqrt(head_dim)) V over positions
 * [0, sequence_length) of the cache layout [kv_head][max_seq][head_dim];
 * head h reads kv head h / (num_heads / num_kv_heads).  scores: scratch of
 * sequence_length floats per thread (threads * max_seq floats). */
void orc_attention_decode(const float* q, const float* key_cache,
                          const float* value_cache, float* output, int num_heads,
                          int num_kv_heads, int head_dim, int sequence_length,
                          int max_sequence_length, int threads);

/* cpu_ops.cpp:168-173: gate / (1 + exp(-gate)) * up. */
void orc_silu_mul(const float* gate, const float* up, float* output, int n);

/* A Qwen2 model on FP32 weights.  Layer-stacked arrays: layer l of a kind
 * starts at l * (its per-layer size).  Biases are q/k/v only (NULL allowed:
 * zero).  The LM head is tied to the embedding. */
typedef struct orc_model_weights {
  const float* embed;       /* [vocab, hidden] */
  const float* final_norm;  /* [hidden] */
  const float* in_norm;     /* [layers][hidden] */
  const float* post_norm;   /* [layers][hidden] */
  const float* wq;          /* [layers][hidden, hidden] */
  const float* bq;          /* [layers][hidden] */
  const float* wk;          /* [layers][kv_dim, hidden] */
  const float* bk;          /* [layers][kv_dim] */
  const float* wv;          /* [layers][kv_dim, hidden] */
  const float* bv;          /* [layers][kv_dim] */
  const float* wo;          /* [layers][hidden, hidden] */
  const float* wg;          /* [layers][inter, hidden] */
  const float* wu;          /* [layers][inter, hidden] */
  const float* wd;          /* [layers][hidden, inter] */
} orc_model_weights;

typedef struct orc_model_config {
  int layers;
  int hidden;
  int heads;
  int kv_heads;
  int inter;
  int vocab;
  int max_seq;
  float eps;
  float theta;
  int threads;
} orc_model_config;

typedef struct orc_model orc_model;

/* Allocates the FP32 KV cache and activations (returns NULL on bad shapes or
 * out of memory).  The weights are borrowed and must outlive the model. */
orc_model* orc_model_create(const orc_model_config* config,
                            const orc_model_weights* weights);
void orc_model_destroy(orc_model* model);

/* qwen2.cpp:427-494: positions [0, count) from tokens; the cache is
 * overwritten from position 0.  logits (vocab floats, may be NULL) gets
 * the last token's logits.  Returns the argmax, or -1 on bad input. */
int orc_model_prefill(orc_model* model, const int* tokens, int count,
                      float* logits);

/* qwen2.cpp:376-425: one token at `position` (the cache holds positions
 * [0, position)).  Returns the argmax, or -1 on bad input. */
int orc_model_decode(orc_model* model, int token, int position, float* logits);

#ifdef __cplusplus
}
#endif

#endif /* MODEL_ORACLE_H */
