// Internal launch interface of the non-Linear decode/prefill kernels
// (model_kernels.hip) used by the model runtime (model.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace qlin {

// Decode state kept in device memory so that a decode step needs no host
// input: `token` is the input of the next step (the LM head's argmax writes
// it), `pos` that token's position, `step` the index of the next history
// entry.
struct ModelState {
  int token;
  int pos;
  int step;
  int pad;
};

// Head dimensions the attention kernels are built for.
bool attention_head_dim_supported(int head_dim);

void launch_embedding(const uint16_t* table, const int* tokens, int count, int vocab, int hidden,
                      uint16_t* out, hipStream_t stream);
void launch_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* out, int rows, int hidden,
                     float eps, hipStream_t stream);
void launch_rope_store(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* key_cache,
                       uint16_t* value_cache, const float2* rope, int count, int start,
                       int heads, int kv_heads, int head_dim, int max_seq, hipStream_t stream);
// Decode attention split over the context (see attention_decode_kernel):
// one workgroup per (span, query head), spans of attention_span(max_seq)
// positions, at most attention_splits(max_seq) of them; partial holds
// heads x attention_splits() x (head_dim + 2) floats.
constexpr int kAttnWaves = 2;
constexpr int kAttnMaxSplits = 8;
int attention_span(int max_seq);
int attention_splits(int max_seq);
void launch_attention_decode(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                             uint16_t* key_cache, uint16_t* value_cache, const float2* rope,
                             const ModelState* state, int heads, int kv_heads, int head_dim,
                             int max_seq, float* partial, hipStream_t stream);
void launch_attention_prefill(const uint16_t* q, const uint16_t* key_cache,
                              const uint16_t* value_cache, uint16_t* out, int count, int heads,
                              int kv_heads, int head_dim, int max_seq, hipStream_t stream);
void launch_silu_mul(const uint16_t* gate, const uint16_t* up, uint16_t* out, long long n,
                     hipStream_t stream);
void launch_add(uint16_t* x, const uint16_t* y, long long n, hipStream_t stream);
// x += y (BF16, in place) and out = rms_norm(x) * w, rows of hidden <= 4096.
void launch_add_rms_norm(uint16_t* x, const uint16_t* y, const uint16_t* w, uint16_t* out,
                         int rows, int hidden, float eps, hipStream_t stream);
void launch_set_state(ModelState* state, int token, int pos, int step, hipStream_t stream);
void launch_advance(ModelState* state, int* history, int history_len, hipStream_t stream);

}  // namespace qlin
