// C ABI of the fused decode-step operators (include/infer_decode.h): the
// kernels of decode_kernels.hip, launched exactly as the model's decode step
// launches them (same rows per wave, grids and kernel instantiations), on
// caller-owned memory.  Each Linear-bearing operator has a W8A16 entry point
// (int8 weights, BF16 group-64 scales) and a BF16 one; both go through one
// implementation here that takes the weight format.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "decode_kernels.hpp"
#include "infer_decode.h"
#include "model_kernels.hpp"
#include "status.hpp"

using namespace qlin;

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Byte layout of the LM-head workspace: the finishing counter, then one
// (value, index) pair per workgroup.
constexpr size_t kLmCounterBytes = 256;

// Weights per 16-byte chunk: 16 int8 or 8 BF16.
int chunk_values(bool w8) { return w8 ? 16 : 8; }

int check_norm_input(const uint16_t* input, const uint16_t* norm_weight, int in_features,
                     bool w8, const char* what) {
  if (!input || !norm_weight) return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null input", what);
  if (!aligned16(input) || !aligned16(norm_weight)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: input and norm weight must be 16-byte aligned",
                what);
  }
  if (!norm_gemv_supported(in_features, w8)) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "%s: in_features %d must be a multiple of 64 in [64, %d]", what, in_features,
                64 * chunk_values(w8) * kNormGemvMaxSlabs);
  }
  return INFER_HIP_OK;
}

// A Linear's weight (and, for W8A16, its scales) and output.
int check_weight(const void* w, const uint16_t* s, bool w8, const void* out, int n,
                 const char* what) {
  if (!w || (w8 && !s) || !out) return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null pointer", what);
  if (!aligned16(w)) return fail(INFER_HIP_INVALID_ARGUMENT, "%s: weight not 16-byte aligned", what);
  if (n < 1) return fail(INFER_HIP_INVALID_ARGUMENT, "%s: out_features %d < 1", what, n);
  return INFER_HIP_OK;
}

// One GEMV of rms_norm_gemv in either format.
struct NormGemvIn {
  const void* weight;
  const uint16_t* scales;
  const uint16_t* bias;
  uint16_t* output;
  int out_features;
};

int rms_norm_gemv(const uint16_t* input, const uint16_t* norm_weight, float epsilon,
                  int in_features, const NormGemvIn* gemvs, int count, bool w8,
                  hipStream_t stream, const char* what) {
  int rc = check_norm_input(input, norm_weight, in_features, w8, what);
  if (rc != INFER_HIP_OK) return rc;
  if (count < 1 || count > kNormGemvMaxDescs) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: count %d must be in [1, %d]", what, count,
                kNormGemvMaxDescs);
  }
  NormGemvArgs a{input, norm_weight, epsilon, in_features, count, kQkvRowsPerWave, {}};
  int blocks = 0;
  for (int i = 0; i < count; ++i) {
    const NormGemvIn& g = gemvs[i];
    rc = check_weight(g.weight, g.scales, w8, g.output, g.out_features, what);
    if (rc != INFER_HIP_OK) return rc;
    a.d[i] = NormGemvDesc{g.weight, w8 ? g.scales : nullptr, nullptr, nullptr, g.bias,
                          g.output, g.out_features, blocks};
    blocks += norm_gemv_blocks(g.out_features, kQkvRowsPerWave);
  }
  launch_norm_gemv(a, blocks, false, w8, stream);
  return check_launch(what);
}

int rms_norm_gate_up_silu(const uint16_t* input, const uint16_t* norm_weight, float epsilon,
                          int in_features, const void* gate_weight, const uint16_t* gate_scales,
                          const void* up_weight, const uint16_t* up_scales, uint16_t* output,
                          int intermediate_size, bool w8, hipStream_t stream,
                          const char* what) {
  int rc = check_norm_input(input, norm_weight, in_features, w8, what);
  if (rc == INFER_HIP_OK) {
    rc = check_weight(gate_weight, gate_scales, w8, output, intermediate_size, what);
  }
  if (rc == INFER_HIP_OK) rc = check_weight(up_weight, up_scales, w8, output, intermediate_size, what);
  if (rc != INFER_HIP_OK) return rc;
  // the row pairs per wave of the model's decode step for this format
  const int rows = w8 ? kGateUpRowsPerWave : kGateUpRowsPerWaveBf16;
  NormGemvArgs a{input, norm_weight, epsilon, in_features, 1, rows, {}};
  a.d[0] = NormGemvDesc{gate_weight, w8 ? gate_scales : nullptr, up_weight,
                        w8 ? up_scales : nullptr, nullptr, output, intermediate_size, 0};
  launch_norm_gemv(a, norm_gemv_blocks(intermediate_size, rows), true, w8, stream);
  return check_launch(what);
}

// One of q, k, v of rms_norm_qkv_rope in either format.
struct QkvWeightIn {
  const void* weight;
  const uint16_t* scales;
  const uint16_t* bias;
};

int rms_norm_qkv_rope(const uint16_t* input, const uint16_t* norm_weight, float epsilon,
                      int in_features, const QkvWeightIn& q_proj, const QkvWeightIn& k_proj,
                      const QkvWeightIn& v_proj, uint16_t* q_out, uint16_t* key_cache,
                      uint16_t* value_cache, const float* rope_row, const int* position,
                      int num_heads, int num_kv_heads, int head_dim, int max_sequence_length,
                      bool w8, hipStream_t stream, const char* what) {
  int rc = check_norm_input(input, norm_weight, in_features, w8, what);
  if (rc != INFER_HIP_OK) return rc;
  if (!q_out || !key_cache || !value_cache || !rope_row || !position) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null pointer", what);
  }
  if (num_heads < 1 || num_kv_heads < 1 || num_heads % num_kv_heads != 0 || head_dim < 2 ||
      head_dim % 2 != 0 || max_sequence_length < 1 ||
      !norm_qkv_rope_supported(in_features, head_dim, w8)) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "%s: bad shape (heads %d, kv heads %d, head_dim %d, max_seq %d, in %d)", what,
                num_heads, num_kv_heads, head_dim, max_sequence_length, in_features);
  }
  const int nq = num_heads * head_dim, nkv = num_kv_heads * head_dim;
  rc = check_weight(q_proj.weight, q_proj.scales, w8, q_out, nq, what);
  if (rc == INFER_HIP_OK) {
    rc = check_weight(k_proj.weight, k_proj.scales, w8, key_cache, nkv, what);
  }
  if (rc == INFER_HIP_OK) {
    rc = check_weight(v_proj.weight, v_proj.scales, w8, value_cache, nkv, what);
  }
  if (rc != INFER_HIP_OK) return rc;
  const QkvRopeArgs a{input, norm_weight, epsilon, in_features,
                      q_proj.weight, w8 ? q_proj.scales : nullptr, q_proj.bias,
                      k_proj.weight, w8 ? k_proj.scales : nullptr, k_proj.bias,
                      v_proj.weight, w8 ? v_proj.scales : nullptr, v_proj.bias,
                      q_out, key_cache, value_cache, reinterpret_cast<const float2*>(rope_row),
                      position, num_heads, num_kv_heads, head_dim, max_sequence_length};
  launch_norm_qkv_rope(a, w8, stream);
  return check_launch(what);
}

int attention_parts_o_proj(const float* records, const int* position, int num_heads,
                           int max_sequence_length, int num_parts, const void* weight,
                           const uint16_t* scales, uint16_t* residual, int out_features,
                           bool w8, hipStream_t stream, const char* what) {
  if (!records || !position || !weight || (w8 && !scales) || !residual) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null pointer", what);
  }
  if (num_parts != 2 && num_parts != 4) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: num_parts %d (2 or 4)", what, num_parts);
  }
  const int in_features = num_heads * 64;
  if (num_heads < 1 || out_features < 1 || max_sequence_length < 1 ||
      max_sequence_length > kAttnWholeMax || !attn_o_parts_supported(in_features, w8)) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "%s: %d heads (in_features %d: multiple of 64, at most %d), %d outputs, "
                "max_sequence_length %d (at most %d)",
                what, num_heads, in_features, 256 * chunk_values(w8), out_features,
                max_sequence_length, kAttnWholeMax);
  }
  if (!aligned16(records) || !aligned16(weight)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: records and weight must be 16-byte aligned",
                what);
  }
  launch_attn_o_parts({records, position, num_heads, max_sequence_length, weight,
                       w8 ? scales : nullptr, residual, out_features, in_features},
                      w8, stream, num_parts);
  return check_launch(what);
}

int gemv_rows(const void* weight, const uint16_t* scales, const uint16_t* bias,
              const uint16_t* input, uint16_t* output, int out_features, int in_features,
              bool w8, hipStream_t stream, const char* what) {
  int rc = check_weight(weight, scales, w8, output, out_features, what);
  if (rc != INFER_HIP_OK) return rc;
  if (!input || !aligned16(input)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: input null or not 16-byte aligned", what);
  }
  if (!gemv_rows_supported(in_features, w8)) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "%s: in_features %d must be a multiple of 64 in [64, %d]", what, in_features,
                w8 ? 8192 : 5120);
  }
  launch_gemv_rows({weight, w8 ? scales : nullptr, bias, input, output, out_features,
                    in_features},
                   w8, stream);
  return check_launch(what);
}

}  // namespace

extern "C" int infer_hip_rms_norm_gemv_w8a16(const uint16_t* input, const uint16_t* norm_weight,
                                             float epsilon, int in_features,
                                             const infer_hip_norm_gemv* gemvs, int count,
                                             hipStream_t stream) {
  const char* what = "rms_norm_gemv_w8a16";
  if (!gemvs) return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null gemvs", what);
  NormGemvIn in[kNormGemvMaxDescs] = {};
  for (int i = 0; i < count && i < kNormGemvMaxDescs; ++i) {
    in[i] = NormGemvIn{gemvs[i].weight, gemvs[i].scales, gemvs[i].bias, gemvs[i].output,
                       gemvs[i].out_features};
  }
  return rms_norm_gemv(input, norm_weight, epsilon, in_features, in, count, true, stream, what);
}

extern "C" int infer_hip_rms_norm_gemv_bf16(const uint16_t* input, const uint16_t* norm_weight,
                                            float epsilon, int in_features,
                                            const infer_hip_norm_gemv_bf16* gemvs, int count,
                                            hipStream_t stream) {
  const char* what = "rms_norm_gemv_bf16";
  if (!gemvs) return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null gemvs", what);
  NormGemvIn in[kNormGemvMaxDescs] = {};
  for (int i = 0; i < count && i < kNormGemvMaxDescs; ++i) {
    in[i] = NormGemvIn{gemvs[i].weight, nullptr, gemvs[i].bias, gemvs[i].output,
                       gemvs[i].out_features};
  }
  return rms_norm_gemv(input, norm_weight, epsilon, in_features, in, count, false, stream, what);
}

extern "C" int infer_hip_rms_norm_gate_up_silu_w8a16(
    const uint16_t* input, const uint16_t* norm_weight, float epsilon, int in_features,
    const int8_t* gate_weight, const uint16_t* gate_scales, const int8_t* up_weight,
    const uint16_t* up_scales, uint16_t* output, int intermediate_size, hipStream_t stream) {
  return rms_norm_gate_up_silu(input, norm_weight, epsilon, in_features, gate_weight,
                               gate_scales, up_weight, up_scales, output, intermediate_size,
                               true, stream, "rms_norm_gate_up_silu_w8a16");
}

extern "C" int infer_hip_rms_norm_gate_up_silu_bf16(
    const uint16_t* input, const uint16_t* norm_weight, float epsilon, int in_features,
    const uint16_t* gate_weight, const uint16_t* up_weight, uint16_t* output,
    int intermediate_size, hipStream_t stream) {
  return rms_norm_gate_up_silu(input, norm_weight, epsilon, in_features, gate_weight, nullptr,
                               up_weight, nullptr, output, intermediate_size, false, stream,
                               "rms_norm_gate_up_silu_bf16");
}

static int attention_decode_parts(const uint16_t* q, const uint16_t* key_cache,
                                  const uint16_t* value_cache, const int* position,
                                  float* records, int num_heads, int num_kv_heads, int head_dim,
                                  int max_sequence_length, int num_parts, hipStream_t stream,
                                  const char* what) {
  if (!q || !key_cache || !value_cache || !position || !records) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null pointer", what);
  }
  if (num_parts != 2 && num_parts != 4) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: num_parts %d (2 or 4)", what, num_parts);
  }
  if (num_heads < 1 || num_kv_heads < 1 || num_heads % num_kv_heads != 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: %d heads, %d kv heads", what, num_heads,
                num_kv_heads);
  }
  if (max_sequence_length < 1 || !attention_whole(max_sequence_length, head_dim)) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "%s: head_dim %d, max_sequence_length %d (head_dim 64, at most %d)", what,
                head_dim, max_sequence_length, kAttnWholeMax);
  }
  if (!aligned16(q) || !aligned16(key_cache) || !aligned16(value_cache) ||
      !aligned16(records)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: q, caches and records must be 16-byte aligned",
                what);
  }
  launch_attention_decode_parts(q, key_cache, value_cache, position, num_heads, num_kv_heads,
                                max_sequence_length, records, stream, num_parts);
  return check_launch(what);
}

extern "C" int infer_hip_attention_decode_halves_bf16(
    const uint16_t* q, const uint16_t* key_cache, const uint16_t* value_cache,
    const int* position, float* records, int num_heads, int num_kv_heads, int head_dim,
    int max_sequence_length, hipStream_t stream) {
  return attention_decode_parts(q, key_cache, value_cache, position, records, num_heads,
                                num_kv_heads, head_dim, max_sequence_length, 2, stream,
                                "attention_decode_halves_bf16");
}

extern "C" int infer_hip_attention_decode_parts_bf16(
    const uint16_t* q, const uint16_t* key_cache, const uint16_t* value_cache,
    const int* position, float* records, int num_heads, int num_kv_heads, int head_dim,
    int max_sequence_length, int num_parts, hipStream_t stream) {
  return attention_decode_parts(q, key_cache, value_cache, position, records, num_heads,
                                num_kv_heads, head_dim, max_sequence_length, num_parts, stream,
                                "attention_decode_parts_bf16");
}

extern "C" int infer_hip_attention_halves_o_proj_w8a16(
    const float* records, const int* position, int num_heads, int max_sequence_length,
    const int8_t* weight, const uint16_t* scales, uint16_t* residual, int out_features,
    hipStream_t stream) {
  return attention_parts_o_proj(records, position, num_heads, max_sequence_length, 2, weight,
                                scales, residual, out_features, true, stream,
                                "attention_halves_o_proj_w8a16");
}

extern "C" int infer_hip_attention_halves_o_proj_bf16(
    const float* records, const int* position, int num_heads, int max_sequence_length,
    const uint16_t* weight, uint16_t* residual, int out_features, hipStream_t stream) {
  return attention_parts_o_proj(records, position, num_heads, max_sequence_length, 2, weight,
                                nullptr, residual, out_features, false, stream,
                                "attention_halves_o_proj_bf16");
}

extern "C" int infer_hip_attention_parts_o_proj_w8a16(
    const float* records, const int* position, int num_heads, int max_sequence_length,
    int num_parts, const int8_t* weight, const uint16_t* scales, uint16_t* residual,
    int out_features, hipStream_t stream) {
  return attention_parts_o_proj(records, position, num_heads, max_sequence_length, num_parts,
                                weight, scales, residual, out_features, true, stream,
                                "attention_parts_o_proj_w8a16");
}

extern "C" int infer_hip_attention_parts_o_proj_bf16(
    const float* records, const int* position, int num_heads, int max_sequence_length,
    int num_parts, const uint16_t* weight, uint16_t* residual, int out_features,
    hipStream_t stream) {
  return attention_parts_o_proj(records, position, num_heads, max_sequence_length, num_parts,
                                weight, nullptr, residual, out_features, false, stream,
                                "attention_parts_o_proj_bf16");
}

extern "C" int infer_hip_gemv_w8a16_rows(const int8_t* weight, const uint16_t* scales,
                                         const uint16_t* bias, const uint16_t* input,
                                         uint16_t* output, int out_features, int in_features,
                                         hipStream_t stream) {
  return gemv_rows(weight, scales, bias, input, output, out_features, in_features, true, stream,
                   "gemv_w8a16_rows");
}

extern "C" int infer_hip_gemv_bf16_rows(const uint16_t* weight, const uint16_t* bias,
                                        const uint16_t* input, uint16_t* output,
                                        int out_features, int in_features, hipStream_t stream) {
  return gemv_rows(weight, nullptr, bias, input, output, out_features, in_features, false,
                   stream, "gemv_bf16_rows");
}

extern "C" int infer_hip_attention_decode_spans_bf16(
    const uint16_t* q, const uint16_t* key_cache, const uint16_t* value_cache,
    const int* position, float* partials, int num_heads, int num_kv_heads, int head_dim,
    int max_sequence_length, hipStream_t stream) {
  const char* what = "attention_decode_spans_bf16";
  if (!q || !key_cache || !value_cache || !position || !partials) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null pointer", what);
  }
  if (num_heads < 1 || num_kv_heads < 1 || num_heads % num_kv_heads != 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: %d heads, %d kv heads", what, num_heads,
                num_kv_heads);
  }
  if (!attention_head_dim_supported(head_dim) || max_sequence_length < 1) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "%s: head_dim %d (64 or 128), max_sequence_length %d", what, head_dim,
                max_sequence_length);
  }
  if (!aligned16(key_cache) || !aligned16(value_cache)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: caches must be 16-byte aligned", what);
  }
  if (2ll * num_kv_heads * max_sequence_length * head_dim >= 0x7FFFFFFFll) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: caches over 2 GiB", what);
  }
  launch_attention_decode_spans(q, key_cache, value_cache, position, num_heads, num_kv_heads,
                                head_dim, max_sequence_length, partials, stream);
  return check_launch(what);
}

extern "C" int infer_hip_attention_decode_span(int max_sequence_length, int head_dim) {
  if (max_sequence_length < 1 || !attention_head_dim_supported(head_dim)) return 0;
  return attention_span(max_sequence_length, head_dim);
}

extern "C" int infer_hip_attention_decode_splits(int max_sequence_length, int head_dim) {
  if (max_sequence_length < 1 || !attention_head_dim_supported(head_dim)) return 0;
  return attention_splits(max_sequence_length, head_dim);
}

extern "C" int infer_hip_attention_merge_o_proj(const float* partials, const int* position,
                                                int num_heads, int head_dim, int span,
                                                int max_splits, int max_sequence_length,
                                                const void* weight, const uint16_t* scales,
                                                uint16_t* residual, int out_features,
                                                hipStream_t stream) {
  const char* what = "attention_merge_o_proj";
  if (!partials || !position || !weight || !residual) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null pointer", what);
  }
  if (!attention_head_dim_supported(head_dim) || num_heads < 1) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: head_dim %d (64 or 128), num_heads %d", what,
                head_dim, num_heads);
  }
  if (max_sequence_length < 1 || span != attention_span(max_sequence_length, head_dim) ||
      max_splits != attention_splits(max_sequence_length, head_dim)) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "%s: span %d / splits %d do not match max_sequence_length %d", what, span,
                max_splits, max_sequence_length);
  }
  const bool w8 = scales != nullptr;
  const int k = num_heads * head_dim;
  if (!attn_o_supported(k, num_heads, w8)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: %d heads x %d is not supported", what,
                num_heads, head_dim);
  }
  if (!aligned16(weight)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: weight not 16-byte aligned", what);
  }
  if (out_features < 1) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: out_features %d < 1", what, out_features);
  }
  launch_attn_o_gemv({partials, position, num_heads, head_dim, span, max_splits,
                      max_sequence_length, weight, scales, residual, out_features, k},
                     w8, stream);
  return check_launch(what);
}

extern "C" size_t infer_hip_lm_head_decode_workspace_bytes(int vocab) {
  if (vocab < 1) return 0;
  return kLmCounterBytes + 8 * static_cast<size_t>(lm_head_decode_blocks(vocab));
}

extern "C" int infer_hip_rms_norm_lm_head_argmax(const uint16_t* input,
                                                 const uint16_t* norm_weight, float epsilon,
                                                 const uint16_t* weight, int vocab,
                                                 int in_features, uint16_t* logits,
                                                 void* workspace, int* argmax,
                                                 hipStream_t stream) {
  const char* what = "rms_norm_lm_head_argmax";
  if (!input || !norm_weight || !weight || !logits || !workspace || !argmax) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null pointer", what);
  }
  if (!aligned16(input) || !aligned16(norm_weight) || !aligned16(weight) ||
      !aligned16(workspace)) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "%s: input, norm weight, weight and workspace must be 16-byte aligned", what);
  }
  if (vocab < 1 || !lm_head_decode_supported(in_features)) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "%s: vocab %d, in_features %d (a multiple of 8 in [8, %d])", what, vocab,
                in_features, 512 * kLmHeadMaxSlabs);
  }
  char* ws = static_cast<char*>(workspace);
  launch_lm_head_decode({input, norm_weight, epsilon, weight, vocab, in_features, logits,
                         reinterpret_cast<float*>(ws + kLmCounterBytes),
                         reinterpret_cast<int*>(ws), argmax, nullptr, nullptr, 0, 0,
                         RopeCursor{nullptr, nullptr, 0, 0}},
                        stream);
  return check_launch(what);
}

extern "C" int infer_hip_rms_norm_qkv_rope_w8a16(
    const uint16_t* input, const uint16_t* norm_weight, float epsilon, int in_features,
    const infer_hip_w8a16_weight* q_proj, const infer_hip_w8a16_weight* k_proj,
    const infer_hip_w8a16_weight* v_proj, uint16_t* q_out, uint16_t* key_cache,
    uint16_t* value_cache, const float* rope_row, const int* position, int num_heads,
    int num_kv_heads, int head_dim, int max_sequence_length, hipStream_t stream) {
  const char* what = "rms_norm_qkv_rope_w8a16";
  if (!q_proj || !k_proj || !v_proj) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null pointer", what);
  }
  return rms_norm_qkv_rope(input, norm_weight, epsilon, in_features,
                           {q_proj->weight, q_proj->scales, q_proj->bias},
                           {k_proj->weight, k_proj->scales, k_proj->bias},
                           {v_proj->weight, v_proj->scales, v_proj->bias}, q_out, key_cache,
                           value_cache, rope_row, position, num_heads, num_kv_heads, head_dim,
                           max_sequence_length, true, stream, what);
}

extern "C" int infer_hip_rms_norm_qkv_rope_bf16(
    const uint16_t* input, const uint16_t* norm_weight, float epsilon, int in_features,
    const infer_hip_bf16_weight* q_proj, const infer_hip_bf16_weight* k_proj,
    const infer_hip_bf16_weight* v_proj, uint16_t* q_out, uint16_t* key_cache,
    uint16_t* value_cache, const float* rope_row, const int* position, int num_heads,
    int num_kv_heads, int head_dim, int max_sequence_length, hipStream_t stream) {
  const char* what = "rms_norm_qkv_rope_bf16";
  if (!q_proj || !k_proj || !v_proj) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null pointer", what);
  }
  return rms_norm_qkv_rope(input, norm_weight, epsilon, in_features,
                           {q_proj->weight, nullptr, q_proj->bias},
                           {k_proj->weight, nullptr, k_proj->bias},
                           {v_proj->weight, nullptr, v_proj->bias}, q_out, key_cache,
                           value_cache, rope_row, position, num_heads, num_kv_heads, head_dim,
                           max_sequence_length, false, stream, what);
}

extern "C" int infer_hip_rope_row(float theta, int head_dim, int position, float* out) {
  if (!out || head_dim < 2 || head_dim % 2 != 0 || position < 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "rope_row: bad arguments (head_dim %d, position %d)",
                head_dim, position);
  }
  for (int i = 0; i < head_dim / 2; ++i) {
    const float2 cs = rope_angle(theta, head_dim, position, i);
    out[2 * i] = cs.x;
    out[2 * i + 1] = cs.y;
  }
  return ok();
}

extern "C" int infer_hip_attention_decode_bf16(const uint16_t* q, const uint16_t* key_cache,
                                               const uint16_t* value_cache, const int* position,
                                               uint16_t* output, int num_heads, int num_kv_heads,
                                               int head_dim, int max_sequence_length,
                                               hipStream_t stream) {
  const char* what = "attention_decode_bf16";
  if (!q || !key_cache || !value_cache || !position || !output) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null pointer", what);
  }
  if (num_heads < 1 || num_kv_heads < 1 || num_heads % num_kv_heads != 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: %d heads, %d kv heads", what, num_heads,
                num_kv_heads);
  }
  if (max_sequence_length < 1 || !attention_whole(max_sequence_length, head_dim)) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "%s: head_dim %d, max_sequence_length %d (head_dim 64, at most %d)", what,
                head_dim, max_sequence_length, kAttnWholeMax);
  }
  if (!aligned16(q) || !aligned16(key_cache) || !aligned16(value_cache)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: q and caches must be 16-byte aligned", what);
  }
  launch_attention_decode(q, nullptr, nullptr, const_cast<uint16_t*>(key_cache),
                          const_cast<uint16_t*>(value_cache), nullptr, position, num_heads,
                          num_kv_heads, head_dim, max_sequence_length, true, nullptr, output,
                          stream);
  return check_launch(what);
}
