// Caller side of the Linear boundary: the kernel selection that
// Qwen2Model::linear_cuda_bf16 / linear_cuda_bf16_batch / lm_head_cuda_bf16
// perform (src/qwen2.cpp:231-330, Greedy-cy/qwen2.5-jetson-inference), over
// weights resolved once instead of looked up by name on every call.  A
// model runtime swaps its CUDA dispatch for these to use the HIP backend.
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <vector>

#include "infer/linear_hip.hpp"

namespace infer {

// include/infer/common.hpp:29 (the dtypes a Linear weight can have).
enum class DType { kFloat32, kBFloat16, kInt8 };

// One Linear layer's device tensors, as the archive record plus its
// quantization record (`<name>.scale`, include/infer/archive.hpp:7-11,
// tools/export_model.py:299) describe them.
struct LinearWeight {
  DType dtype{DType::kBFloat16};     // kInt8 -> W8A16, kBFloat16 -> W16A16
  const void* weight{nullptr};       // [out_features, in_features]
  const uint16_t* scales{nullptr};   // W8A16: BF16 [out, ceil(in / group)]
  int group_size{0};                 // W8A16: must be 64
  const uint16_t* bias{nullptr};     // BF16 [out] or null (only q/k/v have one)
  int out_features{0};
  int in_features{0};
};

namespace hip {

// src/qwen2.cpp:231-260: one token.  INT8 weights take the W8A16 GEMV, BF16
// weights the BF16 GEMV; anything else is an error.
inline void linear(const LinearWeight& w, const uint16_t* input, uint16_t* output,
                   hipStream_t stream) {
  if (w.dtype == DType::kInt8) {
    if (!w.scales) throw Error("W8A16 tensor lacks quantization metadata");
    gemv_w8a16(static_cast<const int8_t*>(w.weight), w.scales, w.group_size, w.bias, input,
               output, w.out_features, w.in_features, stream);
  } else if (w.dtype == DType::kBFloat16) {
    gemv_bf16(static_cast<const uint16_t*>(w.weight), w.bias, input, output, w.out_features,
              w.in_features, stream);
  } else {
    throw Error("BF16 linear requires BF16 or INT8 weights");
  }
}

// src/qwen2.cpp:300-330: token_count tokens.
inline void linear_batch(const LinearWeight& w, const uint16_t* input, uint16_t* output,
                         int token_count, hipStream_t stream) {
  if (w.dtype == DType::kInt8) {
    if (!w.scales) throw Error("W8A16 tensor lacks quantization metadata");
    gemm_w8a16(static_cast<const int8_t*>(w.weight), w.scales, w.group_size, w.bias, input,
               output, token_count, w.out_features, w.in_features, stream);
  } else if (w.dtype == DType::kBFloat16) {
    gemm_bf16(static_cast<const uint16_t*>(w.weight), w.bias, input, output, token_count,
              w.out_features, w.in_features, stream);
  } else {
    throw Error("batched BF16 linear requires BF16 or INT8 weights");
  }
}

// Split-K scratch for linear_batch on lone long-K Linears (down_proj),
// sized at set-up for every token count up to max_tokens and every weight
// it will serve (the sum of their sizes); zeroed once.  The token loop
// allocates nothing.
class GemmWorkspace {
 public:
  GemmWorkspace(int max_tokens, const std::vector<const LinearWeight*>& weights) {
    for (const LinearWeight* w : weights) {
      bytes_ += gemm_workspace_bytes(max_tokens, w->out_features, w->in_features);
    }
    if (bytes_ > 0) {
      check_hip(hipMalloc(&data_, bytes_), "hipMalloc");
      check_hip(hipMemset(data_, 0, bytes_), "hipMemset");
    }
  }
  ~GemmWorkspace() {
    if (data_) (void)hipFree(data_);
  }
  GemmWorkspace(const GemmWorkspace&) = delete;
  GemmWorkspace& operator=(const GemmWorkspace&) = delete;
  void* data() const { return data_; }
  size_t bytes() const { return bytes_; }

 private:
  void* data_{nullptr};
  size_t bytes_{0};
};

// linear_batch with a workspace: the same computation, with long-K
// Linears split over K (calls sharing the workspace must not overlap).
inline void linear_batch(const LinearWeight& w, const uint16_t* input, uint16_t* output,
                         int token_count, const GemmWorkspace& ws, hipStream_t stream) {
  if (w.dtype == DType::kInt8) {
    if (!w.scales) throw Error("W8A16 tensor lacks quantization metadata");
    gemm_w8a16(static_cast<const int8_t*>(w.weight), w.scales, w.group_size, w.bias, input,
               output, token_count, w.out_features, w.in_features, ws.data(), ws.bytes(),
               stream);
  } else if (w.dtype == DType::kBFloat16) {
    gemm_bf16(static_cast<const uint16_t*>(w.weight), w.bias, input, output, token_count,
              w.out_features, w.in_features, ws.data(), ws.bytes(), stream);
  } else {
    throw Error("batched BF16 linear requires BF16 or INT8 weights");
  }
}

// The LM head's device scratch, sized as src/qwen2.cpp:191-199 sizes it
// (ceil(vocab / 8) entries of value and index) plus the argmax slot.
// Allocated once at set-up; the token loop allocates nothing.
class LmHeadWorkspace {
 public:
  explicit LmHeadWorkspace(int vocab) : entries_((static_cast<size_t>(vocab) + 7) / 8) {
    check_hip(hipMalloc(&value_, entries_ * sizeof(float)), "hipMalloc");
    check_hip(hipMalloc(&index_, (entries_ + 1) * sizeof(int)), "hipMalloc");
  }
  ~LmHeadWorkspace() {
    if (value_) (void)hipFree(value_);
    if (index_) (void)hipFree(index_);
  }
  LmHeadWorkspace(const LmHeadWorkspace&) = delete;
  LmHeadWorkspace& operator=(const LmHeadWorkspace&) = delete;
  float* block_max_value() const { return value_; }
  int* block_max_index() const { return index_; }
  int* argmax() const { return index_ + entries_; }

 private:
  size_t entries_;
  float* value_{nullptr};
  int* index_{nullptr};
};

// src/qwen2.cpp:262-285: the tied LM head needs BF16 weights; the argmax
// lands in ws.argmax() on the device (the caller copies it out and syncs,
// src/qwen2.cpp:668-673).
inline void lm_head(const LinearWeight& embed, const uint16_t* input, uint16_t* logits,
                    const LmHeadWorkspace& ws, hipStream_t stream) {
  if (embed.dtype != DType::kBFloat16) throw Error("BF16 tied LM head requires bfloat16 weights");
  lm_head_bf16(static_cast<const uint16_t*>(embed.weight), nullptr, input, logits,
               ws.block_max_value(), ws.block_max_index(), ws.argmax(), embed.out_features,
               embed.in_features, stream);
}

// The GEMVs of one decode step that share an input and do not depend on each
// other — q/k/v on the attention norm (src/qwen2.cpp:615-626), gate/up on the
// MLP norm (646-651) — as one grouped launch.  All weights must be INT8.
inline W8A16GemvPlan make_shared_input_plan(const std::vector<const LinearWeight*>& weights,
                                            const uint16_t* input,
                                            const std::vector<uint16_t*>& outputs) {
  if (weights.size() != outputs.size()) throw Error("one output per weight");
  std::vector<infer_hip_w8a16_gemv_desc> descs;
  descs.reserve(weights.size());
  for (size_t i = 0; i < weights.size(); ++i) {
    const LinearWeight& w = *weights[i];
    if (w.dtype != DType::kInt8) throw Error("grouped GEMV plans take INT8 weights only");
    descs.push_back({static_cast<const int8_t*>(w.weight), w.scales, w.group_size, w.bias,
                     input, outputs[i], w.out_features, w.in_features});
  }
  return W8A16GemvPlan(descs);
}

}  // namespace hip
}  // namespace infer
