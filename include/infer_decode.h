/*
 * C ABI of the fused decode-step operators: the kernels the HIP decode
 * runtime (infer_model.h) runs for one token, exposed one by one on
 * caller-owned device memory.
 *
 * No single reference function corresponds to any of them.  Each replaces a
 * short sequence of the reference's per-op calls on the decode path of
 * Qwen2Model::decode_next (src/qwen2.cpp:597-674, Greedy-cy/qwen2.5-jetson-
 * inference) with one launch:
 *
 *   infer_hip_rms_norm_gemv_w8a16      rms_norm_bf16 (include/infer/cuda_ops.hpp:
 *                                      63-65) + gemv_w8a16 (cuda_ops.hpp:47-50)
 *                                      for q, k and v (qwen2.cpp:612-626)
 *   infer_hip_rms_norm_gate_up_silu_w8a16
 *                                      rms_norm_bf16 + gemv_w8a16 (gate, up) +
 *                                      silu_mul_bf16 (cuda_ops.hpp:100-101;
 *                                      qwen2.cpp:643-654)
 *   infer_hip_rms_norm_qkv_rope_w8a16  rms_norm_bf16 + gemv_w8a16 for q, k, v +
 *                                      rope_bf16 + store_kv_bf16 (cuda_ops.hpp:
 *                                      70-79; qwen2.cpp:612-633)
 *   infer_hip_attention_decode_bf16    attention_decode_bf16 (cuda_ops.hpp:86-91;
 *                                      qwen2.cpp:633-636) on rotated q and a
 *                                      cache that holds the token
 *   infer_hip_attention_decode_halves_bf16
 *                                      the same, split into two context halves
 *                                      whose records
 *   infer_hip_attention_halves_o_proj_w8a16
 *                                      merges before gemv_w8a16 (o_proj) +
 *                                      add_inplace_bf16 (qwen2.cpp:633-641)
 *   infer_hip_attention_decode_parts_bf16,
 *   infer_hip_attention_parts_o_proj_w8a16
 *                                      the same pair in two or four parts
 *                                      (the model's decode step: four)
 *   infer_hip_gemv_w8a16_rows          gemv_w8a16 + add_inplace_bf16 (cuda_ops.hpp:
 *                                      98-99) for down_proj and the residual
 *                                      (qwen2.cpp:655-659)
 *   infer_hip_attention_decode_spans_bf16
 *                                      attention_decode_bf16 in context spans
 *                                      (any capacity, head_dim 64 or 128), whose
 *                                      records
 *   infer_hip_attention_merge_o_proj   merges: the merge of a context-split
 *                                      attention_decode_bf16 (cuda_ops.hpp:86-91)
 *                                      + gemv (o_proj) + add_inplace_bf16
 *                                      (qwen2.cpp:633-641)
 *   infer_hip_rms_norm_lm_head_argmax  rms_norm_bf16 + lm_head_bf16
 *                                      (cuda_ops.hpp:42-45; qwen2.cpp:660-667)
 *
 * The _w8a16 operators have _bf16 siblings for BF16 weights (the W16A16
 * decode step, with gemv_bf16, cuda_ops.hpp:24-26, in place of gemv_w8a16):
 * infer_hip_rms_norm_gemv_bf16, infer_hip_rms_norm_gate_up_silu_bf16,
 * infer_hip_rms_norm_qkv_rope_bf16, infer_hip_attention_halves_o_proj_bf16,
 * infer_hip_attention_parts_o_proj_bf16 and infer_hip_gemv_bf16_rows.  They run the same kernels instantiated for
 * 8 BF16 weights per 16-byte chunk instead of 16 int8 ones, so their K
 * limits are half the W8A16 ones.
 *
 * Numerics are those of the unfused ops: the normalised activations are
 * rounded to BF16 as rms_norm_bf16 stores them, gate and up are rounded to
 * BF16 before SiLU-mul, sums are FP32 and outputs BF16 round-to-nearest-
 * even.  Differences, on purpose: a residual add is one rounding,
 * bf16(W x + r), where the reference rounds W x first; the LM-head argmax is
 * over the FP32 sums (ties to the lowest index), as the CPU path's
 * std::max_element (src/cpu_ops.cpp:175-177).
 *
 * Preconditions, checked on the host (status INFER_HIP_INVALID_ARGUMENT):
 * in_features % 64 == 0 for the Linear operators, 16-byte aligned weight,
 * input and norm-weight pointers, and the size limits of each entry point.
 * Every entry point is asynchronous on `stream`, allocates nothing and
 * returns an infer_linear.h status, with the message in
 * infer_hip_last_error on failure.
 */
#ifndef INFER_DECODE_H
#define INFER_DECODE_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#include "infer_linear.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One GEMV of infer_hip_rms_norm_gemv_w8a16 (W8A16, group 64). */
typedef struct infer_hip_norm_gemv {
  const int8_t* weight;   /* int8 [out_features, in_features] */
  const uint16_t* scales; /* BF16 [out_features, in_features / 64] */
  const uint16_t* bias;   /* BF16 [out_features] or NULL */
  uint16_t* output;       /* BF16 [out_features] */
  int out_features;
} infer_hip_norm_gemv;

/* xn = bf16(rms_norm(input) * norm_weight) (src/cpu_ops.cpp:15-21 with the
 * BF16 store of rms_norm_bf16), then for each of the `count` (1..3) GEMVs
 * output = bf16(W xn + bias), one launch.  in_features <= 4096. */
int infer_hip_rms_norm_gemv_w8a16(const uint16_t* input, const uint16_t* norm_weight,
                                  float epsilon, int in_features,
                                  const infer_hip_norm_gemv* gemvs, int count,
                                  hipStream_t stream);

/* One GEMV of infer_hip_rms_norm_gemv_bf16 (BF16 weights). */
typedef struct infer_hip_norm_gemv_bf16 {
  const uint16_t* weight; /* BF16 [out_features, in_features] */
  const uint16_t* bias;   /* BF16 [out_features] or NULL */
  uint16_t* output;       /* BF16 [out_features] */
  int out_features;
} infer_hip_norm_gemv_bf16;

/* infer_hip_rms_norm_gemv_w8a16 on BF16 weights (the W16A16 decode step):
 * output = bf16(W xn + bias).  in_features <= 2048. */
int infer_hip_rms_norm_gemv_bf16(const uint16_t* input, const uint16_t* norm_weight,
                                 float epsilon, int in_features,
                                 const infer_hip_norm_gemv_bf16* gemvs, int count,
                                 hipStream_t stream);

/* xn as above; output[i] = bf16(silu(g) * u) with g = bf16(gate_i . xn),
 * u = bf16(up_i . xn) (src/cpu_ops.cpp:168-173 on BF16 operands), one
 * launch.  in_features <= 4096. */
int infer_hip_rms_norm_gate_up_silu_w8a16(const uint16_t* input, const uint16_t* norm_weight,
                                          float epsilon, int in_features,
                                          const int8_t* gate_weight,
                                          const uint16_t* gate_scales,
                                          const int8_t* up_weight, const uint16_t* up_scales,
                                          uint16_t* output, int intermediate_size,
                                          hipStream_t stream);

/* The same on BF16 gate and up weights ([intermediate_size, in_features]).
 * in_features <= 2048. */
int infer_hip_rms_norm_gate_up_silu_bf16(const uint16_t* input, const uint16_t* norm_weight,
                                         float epsilon, int in_features,
                                         const uint16_t* gate_weight,
                                         const uint16_t* up_weight, uint16_t* output,
                                         int intermediate_size, hipStream_t stream);

/* The decode step's q|k|v launch (W8A16, group 64): xn as above;
 * q = bf16(Wq xn + bq), k = bf16(Wk xn + bk), v = bf16(Wv xn + bv); q and k
 * rotated (pairs (i, i + head_dim / 2) of each head: a c - b s, b c + a s
 * with (c, s) = rope_row[i], the (cos, sin) of the token's position) and
 * rounded to BF16; q_out <- rotated q ([num_heads][head_dim]); row p =
 * min(*position, max_sequence_length - 1) of key_cache / value_cache
 * ([num_kv_heads][max_sequence_length][head_dim] BF16) <- rotated k, v.
 * A negative *position stores nothing in the caches (q_out is still
 * written), as the attention kernels treat it as an empty context.
 * q, k and v weights are [heads x head_dim, in_features] int8 with BF16
 * scales; biases may be NULL.  in_features <= 4096, head_dim even.  One
 * launch. */
typedef struct infer_hip_w8a16_weight {
  const int8_t* weight;   /* int8 [out_features, in_features] */
  const uint16_t* scales; /* BF16 [out_features, in_features / 64] */
  const uint16_t* bias;   /* BF16 [out_features] or NULL */
} infer_hip_w8a16_weight;

int infer_hip_rms_norm_qkv_rope_w8a16(const uint16_t* input, const uint16_t* norm_weight,
                                      float epsilon, int in_features,
                                      const infer_hip_w8a16_weight* q_proj,
                                      const infer_hip_w8a16_weight* k_proj,
                                      const infer_hip_w8a16_weight* v_proj, uint16_t* q_out,
                                      uint16_t* key_cache, uint16_t* value_cache,
                                      const float* rope_row, const int* position,
                                      int num_heads, int num_kv_heads, int head_dim,
                                      int max_sequence_length, hipStream_t stream);

/* The same q|k|v launch on BF16 weights ([heads x head_dim, in_features]).
 * in_features <= 2048. */
typedef struct infer_hip_bf16_weight {
  const uint16_t* weight; /* BF16 [out_features, in_features] */
  const uint16_t* bias;   /* BF16 [out_features] or NULL */
} infer_hip_bf16_weight;

int infer_hip_rms_norm_qkv_rope_bf16(const uint16_t* input, const uint16_t* norm_weight,
                                     float epsilon, int in_features,
                                     const infer_hip_bf16_weight* q_proj,
                                     const infer_hip_bf16_weight* k_proj,
                                     const infer_hip_bf16_weight* v_proj, uint16_t* q_out,
                                     uint16_t* key_cache, uint16_t* value_cache,
                                     const float* rope_row, const int* position,
                                     int num_heads, int num_kv_heads, int head_dim,
                                     int max_sequence_length, hipStream_t stream);

/* (cos, sin) of position * theta^(-2 i / head_dim) for i < head_dim / 2,
 * in FP32 with the CPU path's arithmetic (src/cpu_ops.cpp:38-41):
 * out[2 i] = cos, out[2 i + 1] = sin (host memory, head_dim floats).  The
 * rope_row of infer_hip_rms_norm_qkv_rope_w8a16.  Host only; 0 on success. */
int infer_hip_rope_row(float theta, int head_dim, int position, float* out);

/* Decode attention of the token at p = min(*position, max_sequence_length
 * - 1) (device memory): for each query head h (kv head h / (num_heads /
 * num_kv_heads)) output[h] = bf16(softmax(q[h] K^T / sqrt(head_dim)) V)
 * over the cache rows [0, p], q already rotated ([num_heads][head_dim]
 * BF16), the caches already holding row p (as
 * infer_hip_rms_norm_qkv_rope_w8a16 leaves them).  FP32 softmax and
 * accumulation.  head_dim 64, max_sequence_length <= 1024: one workgroup
 * per head over the whole context.  Rows past p are never summed, whatever
 * they hold. */
int infer_hip_attention_decode_bf16(const uint16_t* q, const uint16_t* key_cache,
                                    const uint16_t* value_cache, const int* position,
                                    uint16_t* output, int num_heads, int num_kv_heads,
                                    int head_dim, int max_sequence_length, hipStream_t stream);

/* The same attention in two halves, as the decode step runs it: for query
 * head h and half sp (positions [512 sp, 512 sp + 512) of [0, p]) one
 * workgroup stores the record records[(h * 2 + sp) * 68 + i]: i < 64 the
 * half's unnormalised sum of e^(score - m) v, i = 64 m (the half's largest
 * score), i = 65 the sum of e^(score - m).  A half past the context stores
 * nothing.  Same preconditions as infer_hip_attention_decode_bf16; records
 * holds num_heads x 2 x 68 floats, 16-byte aligned. */
int infer_hip_attention_decode_halves_bf16(const uint16_t* q, const uint16_t* key_cache,
                                           const uint16_t* value_cache, const int* position,
                                           float* records, int num_heads, int num_kv_heads,
                                           int head_dim, int max_sequence_length,
                                           hipStream_t stream);

/* The decode step's o-projection over those records (attention_decode_bf16
 * + gemv_w8a16 o_proj + add_inplace_bf16, cuda_ops.hpp:86-99, qwen2.cpp:
 * 633-641): with p = min(*position, max_sequence_length - 1), halves
 * S = {0} for p < 512, else {0, 1}, M = max_{sp in S} m_sp,
 *   a[64 h + d] = bf16( sum_sp acc_sp[d] e^(m_sp - M) * (1 / sum_sp l_sp e^(m_sp - M)) ),
 *   residual[n] = bf16(W[n] . a + residual[n]).
 * W8A16 weight [out_features, num_heads * 64] with BF16 group-64 scales;
 * num_heads * 64 <= 4096; a second half outside S is never summed.
 * *position >= 0: the context holds at least the token's own row (for a
 * negative position the attention stores no record, and the output is
 * undefined). */
int infer_hip_attention_halves_o_proj_w8a16(const float* records, const int* position,
                                            int num_heads, int max_sequence_length,
                                            const int8_t* weight, const uint16_t* scales,
                                            uint16_t* residual, int out_features,
                                            hipStream_t stream);

/* The same on a BF16 weight [out_features, num_heads * 64];
 * num_heads * 64 <= 2048. */
int infer_hip_attention_halves_o_proj_bf16(const float* records, const int* position,
                                           int num_heads, int max_sequence_length,
                                           const uint16_t* weight, uint16_t* residual,
                                           int out_features, hipStream_t stream);

/* The attention and its merge in P = num_parts parts (2 or 4) of
 * S = 1024 / P positions, as the model's decode step runs it in four
 * (quarters: a (kv head, quarter) unit per workgroup of 4 waves, twice as
 * many workgroups as halves, each with half the loads).  Part sp holds
 * positions [S sp, S sp + S) of [0, p] and stores the record
 * records[(h * P + sp) * 68 + i] laid out as above; a part past the
 * context stores nothing.  The o-projection merges the parts
 * {0 .. p / S} as infer_hip_attention_halves_o_proj_w8a16 merges the
 * halves; parts past that set are never summed.  num_parts 2 is exactly
 * the halves operators; records hold num_heads x P x 68 floats.  Same
 * preconditions otherwise. */
int infer_hip_attention_decode_parts_bf16(const uint16_t* q, const uint16_t* key_cache,
                                          const uint16_t* value_cache, const int* position,
                                          float* records, int num_heads, int num_kv_heads,
                                          int head_dim, int max_sequence_length,
                                          int num_parts, hipStream_t stream);
int infer_hip_attention_parts_o_proj_w8a16(const float* records, const int* position,
                                           int num_heads, int max_sequence_length,
                                           int num_parts, const int8_t* weight,
                                           const uint16_t* scales, uint16_t* residual,
                                           int out_features, hipStream_t stream);
int infer_hip_attention_parts_o_proj_bf16(const float* records, const int* position,
                                          int num_heads, int max_sequence_length,
                                          int num_parts, const uint16_t* weight,
                                          uint16_t* residual, int out_features,
                                          hipStream_t stream);

/* output[n] = bf16(sum_k q[n,k] s[n,k/64] input[k] + bias[n]) with one
 * wave per output row and the whole row in flight at once.  bias may be
 * NULL or equal to output (the in-place residual add of the decode step:
 * every element is read and then written by the same lane); it must not
 * otherwise overlap output.  in_features <= 8192. */
int infer_hip_gemv_w8a16_rows(const int8_t* weight, const uint16_t* scales,
                              const uint16_t* bias, const uint16_t* input, uint16_t* output,
                              int out_features, int in_features, hipStream_t stream);

/* The same on a BF16 weight [out_features, in_features]:
 * output[n] = bf16(sum_k w[n,k] input[k] + bias[n]).  in_features <= 5120. */
int infer_hip_gemv_bf16_rows(const uint16_t* weight, const uint16_t* bias,
                             const uint16_t* input, uint16_t* output, int out_features,
                             int in_features, hipStream_t stream);

/* The decode attention in context spans, for any KV capacity and head_dim
 * 64 or 128 (the form the decode step runs beyond 1024 positions or at
 * head_dim 128): q rotated ([num_heads][head_dim] BF16), the caches holding
 * rows [0, p], p = min(*position, max_sequence_length - 1), as for
 * infer_hip_attention_decode_bf16.  For query head h and span c <= p / span
 * (span and splits from infer_hip_attention_decode_span / _splits) one
 * workgroup stores the record partials[(h * splits + c) * (head_dim + 2) +
 * i]: i < head_dim the span's unnormalised sum of e^(score - m) v, then m
 * (its largest score) and l (its sum of e^(score - m)); spans past the
 * context store nothing.  infer_hip_attention_merge_o_proj merges them.
 * Rows past p are never summed.  Replaces attention_decode_bf16
 * (cuda_ops.hpp:86-91) for contexts the whole-context entry does not take. */
int infer_hip_attention_decode_spans_bf16(const uint16_t* q, const uint16_t* key_cache,
                                          const uint16_t* value_cache, const int* position,
                                          float* partials, int num_heads, int num_kv_heads,
                                          int head_dim, int max_sequence_length,
                                          hipStream_t stream);

/* Context span and split count of the decode attention at a KV capacity of
 * max_sequence_length positions and head_dim (64 or 128): split i covers
 * positions [i * span, (i + 1) * span).  At head_dim 64 with up to 1024
 * positions the context is covered whole (span 1024, 1 split: the decode
 * step then runs the four parts of infer_hip_attention_decode_parts_bf16);
 * otherwise at most 8 splits, whose partials the o-projection merges.
 * 0 for max_sequence_length < 1 or another head_dim. */
int infer_hip_attention_decode_span(int max_sequence_length, int head_dim);
int infer_hip_attention_decode_splits(int max_sequence_length, int head_dim);

/* Merge of a context-split decode attention, then the o-projection with the
 * residual add:
 *   p     = min(*position, max_sequence_length - 1) (device memory),
 *   S     = p / span + 1 splits,
 *   a[h]  = bf16( sum_{i<S} acc[h,i] e^(m[h,i]-M) / sum_{i<S} l[h,i] e^(m[h,i]-M) ),
 *           M = max_{i<S} m[h,i]   (FP32, per head h and dimension),
 *   residual[n] = bf16(W[n] . a + residual[n]).
 * partials holds num_heads x max_splits records of head_dim + 2 floats:
 * acc[0..head_dim) (the split's unnormalised sum of e^(score - m) v), m
 * (its largest score) and l (its sum of e^(score - m)); records of splits
 * >= S are not read.  weight is [out_features, num_heads * head_dim], int8
 * with BF16 group-64 scales, or BF16 when scales is NULL.  span and
 * max_splits must be infer_hip_attention_decode_span / _splits of
 * (max_sequence_length, head_dim); num_heads <= 32, head_dim 64 or 128. */
int infer_hip_attention_merge_o_proj(const float* partials, const int* position,
                                     int num_heads, int head_dim, int span, int max_splits,
                                     int max_sequence_length, const void* weight,
                                     const uint16_t* scales, uint16_t* residual,
                                     int out_features, hipStream_t stream);

/* Workspace of infer_hip_rms_norm_lm_head_argmax for a vocabulary of `vocab`
 * rows (0 if vocab < 1).  The caller zeroes it once before the first call;
 * every call leaves it zeroed again. */
size_t infer_hip_lm_head_decode_workspace_bytes(int vocab);

/* logits[v] = bf16(E[v] . xn) with xn = bf16(rms_norm(input) * norm_weight),
 * and *argmax = the first index of the largest FP32 sum, one launch; the
 * last workgroup to finish reduces the per-workgroup winners.  weight is
 * BF16 [vocab, in_features]; in_features % 8 == 0 and <= 4096; workspace
 * as above (calls that share a workspace must not overlap). */
int infer_hip_rms_norm_lm_head_argmax(const uint16_t* input, const uint16_t* norm_weight,
                                      float epsilon, const uint16_t* weight, int vocab,
                                      int in_features, uint16_t* logits, void* workspace,
                                      int* argmax, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* INFER_DECODE_H */
