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

// (cos, sin) of position * theta^(-2 i / head_dim), FP32 with the CPU
// path's arithmetic (src/cpu_ops.cpp:38-41); host code.
float2 rope_angle(float theta, int head_dim, int position, int i);

void launch_embedding(const uint16_t* table, const int* tokens, int count, int vocab, int hidden,
                      uint16_t* out, hipStream_t stream);
void launch_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* out, int rows, int hidden,
                     float eps, hipStream_t stream);
// x = the embedding rows of tokens[0 .. count) (launch_embedding) and out =
// their RMSNorm (launch_rms_norm), as one launch where the rows allow it.
void launch_embedding_rms_norm(const uint16_t* table, const int* tokens, int count, int vocab,
                               int hidden, uint16_t* x, const uint16_t* w, uint16_t* out,
                               float eps, hipStream_t stream);
void launch_rope_store(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* key_cache,
                       uint16_t* value_cache, const float2* rope, int count, int start,
                       int heads, int kv_heads, int head_dim, int max_seq, hipStream_t stream);
// Decode attention (see attention_decode_kernel).  roped, head_dim 64 and
// up to kAttnWholeMax positions of KV capacity: one workgroup per query head
// over the whole context, writing the BF16 attention output to out (heads x
// head_dim; the attention_decode_bf16 operator).  Otherwise one workgroup
// per (span, query head), spans of attention_span() positions, at most
// kAttnMaxSplits of them, writing partial (heads x attention_splits() x
// (head_dim + 2) floats) for the o-projection to merge (the decode step of
// models outside the fused kernels' limits, whose attention is never the
// whole form: those have head_dim 128 or more than kAttnWholeMax
// positions).
constexpr int kAttnWaves = 2;
constexpr int kAttnMaxSplits = 8;
constexpr int kAttnWholeMax = 1024;
bool attention_whole(int max_seq, int head_dim);

// The whole-context attention of the fused decode step (rotated q, k and v
// already in the caches) in P parts of kAttnWholeMax / P positions (P = 2
// halves or 4 quarters): each (query head, part) workgroup stores an
// (acc[64], max, sum) record at partial[(head * P + part) *
// kAttnPartRecord], merged by launch_attn_o_parts; a part past the context
// stores nothing.  head_dim 64, max_seq <= kAttnWholeMax.
// Floats per (head, part) record: acc[64], max, sum, 2 pad (16-byte aligned).
constexpr int kAttnPartRecord = 68;
void launch_attention_decode_parts(const uint16_t* q, const uint16_t* key_cache,
                                   const uint16_t* value_cache, const int* pos, int heads,
                                   int kv_heads, int max_seq, float* partial,
                                   hipStream_t stream, int parts = 2);
#ifndef QLIN_ATTN_PARTS
#define QLIN_ATTN_PARTS 4
#endif
// The parts the model's decode step splits the whole-context attention into.
// Measured at config 4 (Qwen2.5-0.5B W8A16, 24 layers): quarters (56
// workgroups of 4 waves over the 8 XCDs) take 3.12 us per layer against
// 3.86 for halves (28 workgroups of 8 waves) and 2.92 for eighths (112
// workgroups of 2 waves); the o-projection's merge grows with the parts
// (2.92 us with quarters, 3.47 with eighths), so quarters give the fastest
// step (2206 tok/s, eighths 2158).
constexpr int kDecodeAttnParts = QLIN_ATTN_PARTS;
static_assert(kDecodeAttnParts == 2 || kDecodeAttnParts == 4, "halves or quarters");
int attention_span(int max_seq, int head_dim);
int attention_splits(int max_seq, int head_dim);
// roped: q is already rotated and the token's k and v are in the caches at
// pos (the whole form where it applies, else the split form); otherwise
// (split form) q and k_new are rotated here and the first query head of
// each kv head stores k_new and v_new at pos.
// pos: the token's position (device memory).
void launch_attention_decode(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                             uint16_t* key_cache, uint16_t* value_cache, const float2* rope,
                             const int* pos, int heads, int kv_heads, int head_dim,
                             int max_seq, bool roped, float* partial, uint16_t* out,
                             hipStream_t stream);
// The split form on a pre-rotated q and caches holding the token (the
// attention_decode_bf16 contract), at any KV capacity: one (acc, max, sum)
// record per (head, span) in partial (heads x attention_splits() x
// (head_dim + 2) floats); spans past the context write nothing.
void launch_attention_decode_spans(const uint16_t* q, const uint16_t* key_cache,
                                   const uint16_t* value_cache, const int* pos, int heads,
                                   int kv_heads, int head_dim, int max_seq, float* partial,
                                   hipStream_t stream);
void launch_attention_prefill(const uint16_t* q, const uint16_t* key_cache,
                              const uint16_t* value_cache, uint16_t* out, int count, int heads,
                              int kv_heads, int head_dim, int max_seq, hipStream_t stream);
// The prefill attention of a short prompt (count <= kPrefillRopeMaxTokens,
// positions 0 .. count - 1) on the q|k|v GEMM's unrotated q, k and v ([count]
// [heads or kv_heads][head_dim]): the RoPE of q and k and the KV-cache store
// done inside the attention launch (launch_rope_store's results), so no
// RoPE launch runs.  False (nothing launched) where it does not apply:
// then launch_rope_store + launch_attention_prefill.
constexpr int kPrefillRopeMaxTokens = 64;
bool attention_prefill_rope(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            uint16_t* key_cache, uint16_t* value_cache, const float2* rope,
                            uint16_t* out, int count, int heads, int kv_heads, int head_dim,
                            int max_seq, hipStream_t stream);
void launch_silu_mul(const uint16_t* gate, const uint16_t* up, uint16_t* out, long long n,
                     hipStream_t stream);
void launch_add(uint16_t* x, const uint16_t* y, long long n, hipStream_t stream);
// x += y (BF16, in place) and out = rms_norm(x) * w, rows of hidden <= 4096.
void launch_add_rms_norm(uint16_t* x, const uint16_t* y, const uint16_t* w, uint16_t* out,
                         int rows, int hidden, float eps, hipStream_t stream);
// The (cos, sin) row of the decode position, kept beside it: whatever sets
// or advances ModelState::pos also copies table[pos] (half pairs) into row,
// so a kernel that rotates at the current position loads a fixed address
// with its other inputs instead of waiting for pos first.  row == nullptr:
// no row is kept.
struct RopeCursor {
  const float2* table;  // [max_seq][half]
  float2* row;          // [half]
  int half;
  int max_seq;
};
// key (may be null): a pending LM-head key (LmHeadDecodeArgs::key) is
// cleared with the state.
void launch_set_state(ModelState* state, int token, int pos, int step, RopeCursor rope,
                      hipStream_t stream, unsigned long long* key = nullptr);
void launch_advance(ModelState* state, int* history, int history_len, RopeCursor rope,
                    hipStream_t stream);

// A decode step's argmax as one 64-bit word that an atomic max folds across
// workgroups: bit 63 set (a key is pending); bits 31-62 the value as an
// ordered unsigned integer, where NaN and -inf (which never win the argmax's
// comparison) order lowest and -0 counts as +0; bits 0-30 0x7FFFFFFF - row,
// so equal values go to the lowest row.  The largest key is the row the
// argmax's comparison (higher value, then lower row) picks.
__host__ __device__ inline unsigned long long lm_pack_key(float v, int row) {
  unsigned int o = 0;
  if (v == v && v != -__builtin_inff()) {
    const unsigned int u = v == 0.0f ? 0u : __builtin_bit_cast(unsigned int, v);
    o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  }
  return (1ull << 63) | (static_cast<unsigned long long>(o) << 31) |
         static_cast<unsigned long long>(0x7FFFFFFF - row);
}
__host__ __device__ inline int lm_key_row(unsigned long long key) {
  return 0x7FFFFFFF - static_cast<int>(key & 0x7FFFFFFFull);
}

// The first launch of a decode step whose previous step deferred its argmax
// to `key`: a pending key is applied — the token, its history entry, step
// and position moved on, the (cos, sin) row of the new position — and
// cleared; then the token's embedding row goes to out (null: the state
// only).  With no key pending it is the embedding of state->token.
struct DecodeEntryArgs {
  const uint16_t* table;  // [vocab, hidden] BF16
  ModelState* state;
  unsigned long long* key;
  int* history;
  int history_len;
  RopeCursor rope;
  int vocab;
  int hidden;
  uint16_t* out;          // [hidden] BF16 or nullptr
};
void launch_decode_entry(const DecodeEntryArgs& a, hipStream_t stream);

}  // namespace qlin
