// Internal launch interface of the fused decode-step kernels
// (decode_kernels.hip) used by the model runtime.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "model_kernels.hpp"

namespace qlin {

// One GEMV of a fused RMSNorm + GEMV launch (W8A16: int8 weights and BF16
// group-64 scales; BF16: BF16 weights, no scales).  Rows are 4 x
// rows_per_wave per workgroup; block_begin is the launch's first workgroup
// for this GEMV.
// With the PAIR form, (w, s) are gate_proj, (w2, s2) up_proj and y the
// SiLU-mul output; bias is unused.
struct NormGemvDesc {
  const void* w;
  const uint16_t* s;
  const void* w2;
  const uint16_t* s2;
  const uint16_t* bias;
  uint16_t* y;
  int n;
  int block_begin;
};

constexpr int kNormGemvMaxDescs = 3;
constexpr int kNormGemvMaxSlabs = 4;  // K <= 4096 int8 or 2048 BF16 weights
// Rows (gate|up: row pairs) per wave of the decode step's fused launches:
// measured at the Qwen2.5-0.5B shapes, two beat one on int8 weights (q|k|v
// 3.26 -> 3.07 us, gate|up 5.14 -> 4.95 us per launch); on BF16 weights
// (rows twice as long) one row pair per wave is fastest (gate|up 5.70 us,
// against 6.02 with two and 7.06 with four).
constexpr int kQkvRowsPerWave = 2;
constexpr int kGateUpRowsPerWave = 2;
constexpr int kGateUpRowsPerWaveBf16 = 1;

struct NormGemvArgs {
  const uint16_t* x;       // [k] BF16 (the residual stream)
  const uint16_t* norm_w;  // [k] BF16 RMSNorm weight
  float eps;
  int k;
  int count;
  int rows_per_wave;  // 1, 2 or 4
  NormGemvDesc d[kNormGemvMaxDescs];
};

// Slabs of 64 16-byte chunks a row of K weights spans (W8A16: 1024
// weights per slab, BF16: 512).
int norm_gemv_slabs(int k, bool w8);
bool norm_gemv_supported(int k, bool w8);
int norm_gemv_blocks(int n, int rows_per_wave);
void launch_norm_gemv(const NormGemvArgs& a, int blocks, bool pair, bool w8,
                      hipStream_t stream);

// The decode step's q|k|v launch with the RoPE and the KV-cache store
// folded in: xn = bf16(rms_norm(x) * norm_w); q = bf16(Wq xn + bq),
// k = bf16(Wk xn + bk), v = bf16(Wv xn + bv); q and k rotated by the angles
// of position *pos (pairs (i, i + head_dim / 2) of a head; rope_row holds
// that position's (cos, sin), see RopeCursor) and rounded to BF16;
// q_out <- rotated q, the caches' row *pos <- rotated k and v.
struct QkvRopeArgs {
  const uint16_t* x;       // [k] BF16 residual stream
  const uint16_t* norm_w;  // [k] BF16 input RMSNorm weight
  float eps;
  int k;
  const void* wq;          // int8 (W8A16) or BF16
  const uint16_t* sq;      // W8A16 group scales, else unused
  const uint16_t* bq;      // [heads * head_dim] or nullptr
  const void* wk;
  const uint16_t* sk;
  const uint16_t* bk;      // [kv_heads * head_dim] or nullptr
  const void* wv;
  const uint16_t* sv;
  const uint16_t* bv;
  uint16_t* q_out;         // [heads * head_dim]
  uint16_t* key_cache;     // the layer's [kv_heads][max_seq][head_dim]
  uint16_t* value_cache;
  const float2* rope_row;  // [head_dim / 2] (cos, sin) of position *pos
  const int* pos;          // position of the token (device)
  int heads;
  int kv_heads;
  int head_dim;
  int max_seq;
};

// Workgroups of a launch (one wave per pair of output rows).
int norm_qkv_rope_blocks(int heads, int kv_heads, int head_dim);
bool norm_qkv_rope_supported(int k, int head_dim, bool w8);
void launch_norm_qkv_rope(const QkvRopeArgs& a, bool w8, hipStream_t stream);

// One GEMV row per wave with the whole row's loads in flight at once:
// y[row] = bf16(W[row] . x + bias[row]), bias may alias y (the residual add).
// K % 64 == 0, 16-byte aligned w and x; K <= 8192 for W8A16 weights, K <=
// 5120 for BF16 weights.
struct GemvRowsArgs {
  const void* w;         // [n, k] int8 (W8A16) or BF16
  const uint16_t* s;     // [n, k / 64] BF16 scales (W8A16)
  const uint16_t* bias;  // [n] BF16 or nullptr
  const uint16_t* x;     // [k] BF16
  uint16_t* y;           // [n] BF16
  int n;
  int k;
};

bool gemv_rows_supported(int k, bool w8);
void launch_gemv_rows(const GemvRowsArgs& a, bool w8, hipStream_t stream);

// o-projection fused with the decode attention's split merge and the
// residual add (x = bf16(Wo attn + x)).
constexpr int kAttnOMaxHeads = 32;

struct AttnOArgs {
  const float* partial;     // heads x max_splits x (head_dim + 2) floats
  const int* pos;           // position of the decoded token (device)
  int heads;
  int head_dim;
  int span;                 // attention_span(max_seq)
  int max_splits;           // attention_splits(max_seq)
  int max_seq;
  const void* w;            // [n, k] int8 (W8A16) or BF16
  const uint16_t* s;        // [n, k / 64] BF16 scales (W8A16)
  uint16_t* x;              // [n] residual stream, updated in place
  int n;
  int k;                    // heads x head_dim
};

bool attn_o_supported(int k, int heads, bool w8);

// The fused decode step's o-projection (W8A16 group 64, or BF16) with the
// merge of the attention's P parts (launch_attention_decode_parts; P = 2
// halves or 4 quarters of S = kAttnWholeMax / P positions):
//   a[i] = bf16( sum_sp acc_sp[i] e^(m_sp - M) / sum_sp l_sp e^(m_sp - M) ),
//   M = max_sp m_sp over the parts [0, pos / S],
//   x[row] = bf16(Wo[row] . a + x[row]).
// Each workgroup merges the k attention outputs once (each thread four of
// them) into BF16 in LDS, shared by its four waves (one output row each)
// after one barrier.
struct AttnOPartsArgs {
  const float* partial;  // heads x P records of kAttnPartRecord floats
  const int* pos;        // position of the decoded token (device)
  int heads;
  int max_seq;
  const void* w;         // [n, k] int8 (W8A16) or BF16
  const uint16_t* s;     // [n, k / 64] BF16 scales (W8A16)
  uint16_t* x;           // [n] residual stream, updated in place
  int n;
  int k;                 // heads x 64
};
bool attn_o_parts_supported(int k, bool w8);
// parts: 2 (the halves' records) or 4 (quarters', as
// launch_attention_decode_parts with parts 4 leaves them).
void launch_attn_o_parts(const AttnOPartsArgs& a, bool w8, hipStream_t stream,
                         int parts = 2);
void launch_attn_o_gemv(const AttnOArgs& a, bool w8, hipStream_t stream);

constexpr int kLmHeadMaxSlabs = 8;  // K <= 4096

struct LmHeadDecodeArgs {
  const uint16_t* x;       // [k] BF16 final hidden state (before the norm)
  const uint16_t* norm_w;  // [k] BF16 final RMSNorm weight
  float eps;
  const uint16_t* w;       // [vocab, k] BF16 (tied embedding)
  int vocab;
  int k;
  uint16_t* logits;        // [vocab] BF16
  float* block_best;       // lm_head_decode_blocks(vocab) (value, index) pairs
  int* counter;            // zero between launches
  int* token;              // the argmax is written here
  ModelState* state;       // with advance: step / pos moved on (else unused)
  int* history;
  int history_len;
  int advance;             // 1: record the token and advance step / pos
  RopeCursor rope;         // with advance 1: the row follows pos
  // advance 2 (the model's decode step): each workgroup folds its best
  // (value, row) into *key with one 64-bit atomic max (lm_pack_key) and
  // nothing else; the next decode_entry_kernel applies it.  counter, token,
  // state, history and rope are then unused.
  unsigned long long* key = nullptr;
  // With x_add ([k] BF16), the row normalized is bf16(x + x_add): the
  // prefill's last residual add, for the one row the LM head reads.
  const uint16_t* x_add = nullptr;
};

constexpr int kLmHeadRows = 4;  // rows per wave task

bool lm_head_decode_supported(int k);
// The grid the model's launches use (block_best holds this many pairs).
int lm_head_decode_blocks(int vocab);
void launch_lm_head_decode(const LmHeadDecodeArgs& a, hipStream_t stream);
// Explicit grid (<= lm_head_decode_blocks(vocab)) and rows per task (1, 2, 4, 8).
void launch_lm_head_decode_shape(const LmHeadDecodeArgs& a, int grid, int rows,
                                 hipStream_t stream);

}  // namespace qlin
