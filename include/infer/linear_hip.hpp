// C++17 face of the MI355X Linear hot path: the operator boundary of
// include/infer/cuda_ops.hpp (Greedy-cy/qwen2.5-jetson-inference) with the
// same names, argument order and meaning, on HIP streams.  BF16 tensors are
// their 16-bit words (uint16_t).  Every function enqueues work on `stream`
// and throws infer::Error where the reference throws (INFER_CHECK /
// INFER_CUDA_CHECK, include/infer/common.hpp:66-82).  Header-only over the C
// ABI of include/infer_linear.h; link with libinfer_linear.so.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "infer_linear.h"

namespace infer {

// include/infer/common.hpp:66-69.
class Error : public std::runtime_error {
 public:
  using std::runtime_error::runtime_error;
};

namespace hip {

inline void check(int status) {
  if (status != INFER_HIP_OK) throw ::infer::Error(infer_hip_last_error());
}

inline void check_hip(hipError_t status, const char* what) {
  if (status != hipSuccess) {
    throw ::infer::Error(std::string(what) + " failed: " + hipGetErrorString(status));
  }
}

// include/infer/cuda_ops.hpp:10-22, kernels.cu:1404-1415: owns one
// non-blocking stream.  There is no BLAS handle: the hot path has one
// backend.
class Context {
 public:
  Context() { check_hip(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate"); }
  ~Context() {
    if (stream_) (void)hipStreamDestroy(stream_);
  }
  Context(const Context&) = delete;
  Context& operator=(const Context&) = delete;
  hipStream_t stream() const { return stream_; }
  void synchronize() const { check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize"); }

 private:
  hipStream_t stream_{nullptr};
};

// cuda_ops.hpp:24-26.
inline void gemv_bf16(const uint16_t* weight, const uint16_t* bias, const uint16_t* input,
                      uint16_t* output, int out_features, int in_features,
                      hipStream_t stream) {
  check(infer_hip_gemv_bf16(weight, bias, input, output, out_features, in_features, stream));
}

// cuda_ops.hpp:32-35.
inline void gemm_bf16(const uint16_t* weight, const uint16_t* bias, const uint16_t* input,
                      uint16_t* output, int tokens, int out_features, int in_features,
                      hipStream_t stream) {
  check(infer_hip_gemm_bf16(weight, bias, input, output, tokens, out_features, in_features,
                            stream));
}

// Entries of each LM-head scratch array (never more than ceil(vocab / 8),
// the reference's sizing at src/qwen2.cpp:193-198).
inline size_t lm_head_workspace_entries(int vocab, int in_features) {
  return infer_hip_lm_head_workspace_entries(vocab, in_features);
}

// cuda_ops.hpp:42-45.  The argmax is over the FP32 sums (ties to the lowest
// index), so it equals the CPU FP32 argmax.
inline void lm_head_bf16(const uint16_t* weight, const uint16_t* bias, const uint16_t* input,
                         uint16_t* logits, float* block_max_value, int* block_max_index,
                         int* argmax, int vocab, int in_features, hipStream_t stream) {
  check(infer_hip_lm_head_bf16(weight, bias, input, logits, block_max_value, block_max_index,
                               argmax, vocab, in_features, stream));
}

// cuda_ops.hpp:47-50.
inline void gemv_w8a16(const int8_t* weight, const uint16_t* scales, int group_size,
                       const uint16_t* bias, const uint16_t* input, uint16_t* output,
                       int out_features, int in_features, hipStream_t stream) {
  check(infer_hip_gemv_w8a16(weight, scales, group_size, bias, input, output, out_features,
                             in_features, stream));
}

// cuda_ops.hpp:51-55.
inline void gemm_w8a16(const int8_t* weight, const uint16_t* scales, int group_size,
                       const uint16_t* bias, const uint16_t* input, uint16_t* output,
                       int tokens, int out_features, int in_features, hipStream_t stream) {
  check(infer_hip_gemm_w8a16(weight, scales, group_size, bias, input, output, tokens,
                             out_features, in_features, stream));
}

// gemm_w8a16 / gemm_bf16 with a caller workspace (infer_hip_gemm_*_ws): a
// lone long-K call splits K over the idle CUs.  No reference counterpart.
inline size_t gemm_workspace_bytes(int max_tokens, int out_features, int in_features) {
  return infer_hip_gemm_workspace_bytes(max_tokens, out_features, in_features);
}
inline void gemm_w8a16(const int8_t* weight, const uint16_t* scales, int group_size,
                       const uint16_t* bias, const uint16_t* input, uint16_t* output,
                       int tokens, int out_features, int in_features, void* workspace,
                       size_t workspace_bytes, hipStream_t stream) {
  check(infer_hip_gemm_w8a16_ws(weight, scales, group_size, bias, input, output, tokens,
                                out_features, in_features, workspace, workspace_bytes, stream));
}
inline void gemm_bf16(const uint16_t* weight, const uint16_t* bias, const uint16_t* input,
                      uint16_t* output, int tokens, int out_features, int in_features,
                      void* workspace, size_t workspace_bytes, hipStream_t stream) {
  check(infer_hip_gemm_bf16_ws(weight, bias, input, output, tokens, out_features, in_features,
                               workspace, workspace_bytes, stream));
}

// A grouped W8A16 GEMV plan (RAII): many independent gemv_w8a16 calls in
// one launch, resolved once.  No single reference counterpart.
class W8A16GemvPlan {
 public:
  explicit W8A16GemvPlan(const std::vector<infer_hip_w8a16_gemv_desc>& descs) {
    check(infer_hip_w8a16_gemv_plan_create(descs.data(), static_cast<int>(descs.size()),
                                           &plan_));
  }
  ~W8A16GemvPlan() {
    if (plan_) (void)infer_hip_w8a16_gemv_plan_destroy(plan_);
  }
  W8A16GemvPlan(const W8A16GemvPlan&) = delete;
  W8A16GemvPlan& operator=(const W8A16GemvPlan&) = delete;
  W8A16GemvPlan(W8A16GemvPlan&& other) noexcept : plan_(std::exchange(other.plan_, nullptr)) {}
  void launch(hipStream_t stream) const { check(infer_hip_w8a16_gemv_plan_launch(plan_, stream)); }
  double bytes() const { return infer_hip_w8a16_gemv_plan_bytes(plan_); }

 private:
  infer_hip_gemv_plan* plan_{nullptr};
};

// A grouped prefill GEMM plan (RAII): many independent gemm_w8a16 (or
// gemm_bf16) calls in one launch, resolved once; long reductions are split
// over K.  No single reference counterpart.
class GemmPlan {
 public:
  explicit GemmPlan(const std::vector<infer_hip_gemm_desc>& descs) {
    check(infer_hip_gemm_plan_create(descs.data(), static_cast<int>(descs.size()), &plan_));
  }
  ~GemmPlan() {
    if (plan_) (void)infer_hip_gemm_plan_destroy(plan_);
  }
  GemmPlan(const GemmPlan&) = delete;
  GemmPlan& operator=(const GemmPlan&) = delete;
  GemmPlan(GemmPlan&& other) noexcept : plan_(std::exchange(other.plan_, nullptr)) {}
  void launch(hipStream_t stream) const { check(infer_hip_gemm_plan_launch(plan_, stream)); }
  double flops() const { return infer_hip_gemm_plan_flops(plan_); }

 private:
  infer_hip_gemm_plan* plan_{nullptr};
};

}  // namespace hip
}  // namespace infer
