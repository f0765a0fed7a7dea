/*
 * C ABI of the HIP (gfx950) Qwen2 decode runtime built around the Linear
 * path: the device-side orchestration of Qwen2Model's BF16 / W8A16 prefill
 * and decode (src/qwen2.cpp:496-674 and the public surface of
 * include/infer/qwen2.hpp:41-67, Greedy-cy/qwen2.5-jetson-inference).
 *
 * Differences from the reference, all on purpose:
 *   - Weights are caller-owned device tensors passed by pointer (the
 *     reference resolves them by name from a QWENBIN1 archive it uploads,
 *     src/qwen2.cpp:56-78); the runtime resolves every pointer once.
 *   - The decode position and current token live in device memory, so a
 *     decode step needs no host input and is replayed from one captured HIP
 *     graph per token; generate() runs its decode loop without a host sync
 *     per token (the reference syncs every token, src/qwen2.cpp:668-673).
 *   - The residual add after o_proj and down_proj is fused into the GEMV:
 *     x = bf16(W a + x) with one rounding, where the reference rounds the
 *     product to BF16 first and then the sum (src/qwen2.cpp:639-642,
 *     656-660).  Both are within the model's BF16 tolerance of the FP32
 *     CPU path.
 *
 * Every entry point that returns int returns a status code of
 * include/infer_linear.h, with the message in infer_hip_last_error.  A
 * model is not thread-safe: one host thread drives it at a time, as the
 * reference's Qwen2Model.
 */
#ifndef INFER_MODEL_H
#define INFER_MODEL_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#include "infer_linear.h"

#ifdef __cplusplus
extern "C" {
#endif

/* include/infer/common.hpp:30 (Precision); kFloat32 is the CPU path. */
enum infer_hip_precision {
  INFER_HIP_PRECISION_W16A16 = 1, /* BF16 weights */
  INFER_HIP_PRECISION_W8A16 = 2   /* int8 group-64 weights, BF16 scales */
};

/* include/infer/model_config.hpp:7-20. */
typedef struct infer_hip_model_config {
  int hidden_size;
  int intermediate_size;
  int num_layers;
  int num_heads;
  int num_kv_heads;
  int vocab_size;
  int eos_token_id; /* -1: none */
  float rms_norm_eps;
  float rope_theta;
} infer_hip_model_config;

/* One Linear: weight [out, in] (int8 under W8A16, else BF16), scales BF16
 * [out, in / 64] (W8A16 only, else NULL), bias BF16 [out] or NULL (the
 * reference has biases on q/k/v only).  Device pointers, 16-byte aligned. */
typedef struct infer_hip_linear {
  const void* weight;
  const uint16_t* scales;
  const uint16_t* bias;
} infer_hip_linear;

/* model.layers.<i>.* of the archive (src/qwen2.cpp:606-660). */
typedef struct infer_hip_layer_weights {
  const uint16_t* input_layernorm;          /* BF16 [hidden] */
  const uint16_t* post_attention_layernorm; /* BF16 [hidden] */
  infer_hip_linear q_proj;                  /* [hidden, hidden] + bias */
  infer_hip_linear k_proj;                  /* [kv_dim, hidden] + bias */
  infer_hip_linear v_proj;                  /* [kv_dim, hidden] + bias */
  infer_hip_linear o_proj;                  /* [hidden, hidden] */
  infer_hip_linear gate_proj;               /* [inter, hidden] */
  infer_hip_linear up_proj;                 /* [inter, hidden] */
  infer_hip_linear down_proj;               /* [hidden, inter] */
} infer_hip_layer_weights;

typedef struct infer_hip_model_weights {
  const uint16_t* embed_tokens; /* BF16 [vocab, hidden] */
  const uint16_t* norm;         /* BF16 [hidden] (model.norm.weight) */
  const uint16_t* lm_head;      /* BF16 [vocab, hidden]; NULL: tied to embed_tokens */
  const infer_hip_layer_weights* layers; /* num_layers entries, host memory */
} infer_hip_model_weights;

/* include/infer/qwen2.hpp:16-21 (RuntimeOptions); the backend is HIP. */
typedef struct infer_hip_runtime_options {
  int precision;           /* infer_hip_precision */
  int max_sequence_length; /* KV-cache capacity in positions */
  int use_graph;           /* nonzero: decode steps replay a captured HIP graph */
} infer_hip_runtime_options;

/* include/infer/qwen2.hpp:23-34 (GenerationStats). */
typedef struct infer_hip_generation_stats {
  int prompt_tokens;
  int generated_tokens;
  double ttft_ms;
  double decode_ms;
  double total_ms;
} infer_hip_generation_stats;

typedef struct infer_hip_model infer_hip_model;

/* Qwen2Model::Qwen2Model (src/qwen2.cpp:30-54, workspace 80-199): validates the shapes
 * (head_dim 64 or 128, at most 32 query heads, hidden <= 4096, K % 64 == 0
 * and 16-byte aligned weights for the fast Linear paths), allocates the KV cache
 * (BF16 [layer][k|v][kv_head][max_seq][head_dim]) and every workspace on
 * the current device, and creates the model's stream.  The weights are
 * borrowed and must outlive the model. */
int infer_hip_model_create(const infer_hip_model_config* config,
                           const infer_hip_model_weights* weights,
                           const infer_hip_runtime_options* options,
                           infer_hip_model** model);
int infer_hip_model_destroy(infer_hip_model* model);

/* Qwen2Model::reset (src/qwen2.cpp:711-714). */
int infer_hip_model_reset(infer_hip_model* model);

/* Qwen2Model::prefill (src/qwen2.cpp:716-734): tokens is host memory;
 * requires a fresh state; writes the argmax of the last token's logits to
 * *next_token (synchronizes).  A one-token prompt runs as the decode step
 * at position 0 (the same launches as decode_next). */
int infer_hip_model_prefill(infer_hip_model* model, const int* tokens, int count,
                            int* next_token);

/* Qwen2Model::decode_next (src/qwen2.cpp:736-743): one step on `token` at
 * the current position; writes the argmax to *next_token (synchronizes). */
int infer_hip_model_decode_next(infer_hip_model* model, int token, int* next_token);

/* Truncates the context to its first `position` positions (their KV-cache
 * rows are kept) and makes `token` the next decode input, at `position`:
 * the state a prefill of those positions leaves, without recomputing it.
 * Requires a prefilled model, 1 <= position <= its position and a token
 * in range; host-side only (no GPU work).  No reference counterpart (the
 * reference can only reset, src/qwen2.cpp:711-714): for decoding again
 * from a shared prompt, e.g. a benchmark that repeats one decode, or for
 * dropping tokens a caller rejects. */
int infer_hip_model_rewind(infer_hip_model* model, int position, int token);

/* Free-running greedy decode: `steps` steps, each feeding the previous
 * step's argmax, starting from the token the last prefill / decode_next
 * returned.  No host synchronization between steps; tokens_out (host, may
 * be NULL) receives the `steps` generated tokens, after one final sync. */
int infer_hip_model_decode_steps(infer_hip_model* model, int steps, int* tokens_out);

/* Qwen2Model::generate (src/qwen2.cpp:745-776): reset, prefill, then
 * decode until max_new_tokens tokens (or EOS when stop_on_eos).  tokens_out
 * (host) holds max_new_tokens entries; *generated gets the count. */
int infer_hip_model_generate(infer_hip_model* model, const int* prompt, int prompt_count,
                             int max_new_tokens, int stop_on_eos, int* tokens_out,
                             int* generated, infer_hip_generation_stats* stats);

/* Qwen2Model::last_logits_host (src/qwen2.cpp:689-709): the BF16 logits
 * of the last prefill / decode step as FP32 (vocab_size floats). */
int infer_hip_model_last_logits(infer_hip_model* model, float* logits);

/* Qwen2Model::position / has_prefilled (include/infer/qwen2.hpp:58-59). */
int infer_hip_model_position(const infer_hip_model* model);
int infer_hip_model_has_prefilled(const infer_hip_model* model);

/* Qwen2Model::kv_cache_bytes / workspace_bytes (include/infer/qwen2.hpp:60-67). */
size_t infer_hip_model_kv_cache_bytes(const infer_hip_model* model);
size_t infer_hip_model_workspace_bytes(const infer_hip_model* model);

/* attention_prefill_bf16 (include/infer/cuda_ops.hpp:92-97, src/cuda/
 * kernels.cu:221-283, 1507-1518): causal attention of token_count queries at
 * positions 0 .. token_count - 1 over caches [num_kv_heads][max_sequence_length]
 * [head_dim] already holding those positions; q and output are
 * [token_count][num_heads][head_dim] BF16, query head h reads kv head
 * h / (num_heads / num_kv_heads).  The kernel the model's prefill runs: MFMA
 * tiles of 32 queries x 32 keys when every pointer is 16-byte aligned, an
 * exact per-query loop otherwise.  head_dim 64 or 128; FP32 softmax and
 * accumulation, BF16 output.  Stream-ordered, no synchronisation. */
int infer_hip_attention_prefill_bf16(const uint16_t* q, const uint16_t* key_cache,
                                     const uint16_t* value_cache, uint16_t* output,
                                     int token_count, int num_heads, int num_kv_heads,
                                     int head_dim, int max_sequence_length, hipStream_t stream);

/* gemm_w8a16 (include/infer/cuda_ops.hpp:51-55) for mlp.gate_proj and
 * mlp.up_proj of one input, then silu_mul_bf16 (cuda_ops.hpp:100-101), as
 * the prefill calls them (src/qwen2.cpp:560-568), in one launch:
 *   output[t][n] = bf16(silu(g) * u),  g = bf16(input[t] . gate[n] + gate_bias[n]),
 *                                      u = bf16(input[t] . up[n] + up_bias[n]),
 * the unfused ops' roundings and SiLU-mul expression.  input [tokens][hidden],
 * gate and up [intermediate][hidden] (W8A16: int8 with BF16 group-64 scales
 * [intermediate][hidden / 64]), output [tokens][intermediate]; biases may be
 * null.  256-token x 64-column tiles of both GEMMs on MFMA, built for prefills
 * of 256 tokens or more (fewer tokens are computed correctly on partly empty
 * tiles).  Needs hidden % 64 == 0 and 16-byte aligned weights and input.
 * Stream-ordered, allocates nothing. */
int infer_hip_gemm_gate_up_silu_w8a16(const int8_t* gate_weight, const uint16_t* gate_scales,
                                      const uint16_t* gate_bias, const int8_t* up_weight,
                                      const uint16_t* up_scales, const uint16_t* up_bias,
                                      int group_size, const uint16_t* input, uint16_t* output,
                                      int tokens, int intermediate, int hidden,
                                      hipStream_t stream);
int infer_hip_gemm_gate_up_silu_bf16(const uint16_t* gate_weight, const uint16_t* gate_bias,
                                     const uint16_t* up_weight, const uint16_t* up_bias,
                                     const uint16_t* input, uint16_t* output, int tokens,
                                     int intermediate, int hidden, hipStream_t stream);

/* The stream every kernel of the model runs on (infer::cuda::Context). */
hipStream_t infer_hip_model_stream(const infer_hip_model* model);

/* Per-kernel timing of the decode step (the HIP counterpart of the
 * reference's NVTX profiling ranges, src/qwen2.cpp:14-24): the launches of
 * each kind in one decode step (e.g. the 24 layers' gate|up GEMVs) are
 * captured as a graph and replayed `reps` times between two HIP events on
 * the model's stream, at the KV-cache context `position` (1 <= position <=
 * the model's position); a kind with fewer than 24 launches per step is
 * captured that many times over, so the graph launch's overhead is shared as
 * in the decode step.  For kind i (0 <= i < INFER_HIP_MODEL_KERNEL_KINDS,
 * names from infer_hip_model_kernel_name): us[i] = microseconds per launch
 * (the kernel plus its share of graph dispatch, as in the decode step),
 * bytes[i] = its compulsory HBM bytes per launch, launches[i] = launches of
 * that kind per decode step (0: the kind does not occur).  The replays
 * overwrite the KV-cache row at `position` and the activations, so the call
 * ends with the model reset (position 0, not prefilled). */
#define INFER_HIP_MODEL_KERNEL_KINDS 9
int infer_hip_model_kernel_times(infer_hip_model* model, int position, int reps, double* us,
                                 double* bytes, int* launches, int count);
const char* infer_hip_model_kernel_name(int kind);

#ifdef __cplusplus
}
#endif

#endif /* INFER_MODEL_H */
