// Prefill (M = tokens > 1) Linear entry points.
#include <stdint.h>

#include "linear_kernels.hpp"
#include "status.hpp"

using namespace qlin;

extern "C" int infer_hip_gemm_w8a16(const int8_t* weight, const uint16_t* scales,
                                    int group_size, const uint16_t* bias,
                                    const uint16_t* input, uint16_t* output, int tokens,
                                    int out_features, int in_features, hipStream_t stream) {
  // kernels.cu:1661 — the only supported group size.
  if (group_size != 64) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "w8a16 group size must be 64 (got %d)", group_size);
  }
  if (tokens <= 0 || out_features <= 0 || in_features < 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemm_w8a16: bad shape M=%d N=%d K=%d", tokens,
                out_features, in_features);
  }
  if (!output || (in_features > 0 && (!weight || !scales || !input))) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemm_w8a16: null required pointer");
  }
  if (tokens == 1 && w8a16_gemv_fast_supported(weight, input, in_features)) {
    launch_w8a16_gemv_fast({weight, scales, bias, input, output, out_features, in_features},
                           stream);
  } else {
    launch_w8a16_linear_generic(weight, scales, group_size, bias, input, output, tokens,
                                out_features, in_features, stream);
  }
  return check_launch("gemm_w8a16");
}

extern "C" int infer_hip_gemm_bf16(const uint16_t* weight, const uint16_t* bias,
                                   const uint16_t* input, uint16_t* output, int tokens,
                                   int out_features, int in_features, hipStream_t stream) {
  if (tokens <= 0 || out_features <= 0 || in_features < 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemm_bf16: bad shape M=%d N=%d K=%d", tokens,
                out_features, in_features);
  }
  if (!output || (in_features > 0 && (!weight || !input))) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemm_bf16: null required pointer");
  }
  if (tokens == 1 && bf16_gemv_fast_supported(weight, input, in_features)) {
    launch_bf16_gemv_fast({weight, bias, input, output, out_features, in_features}, stream);
  } else {
    launch_bf16_linear_generic(weight, bias, input, output, tokens, out_features, in_features,
                               stream);
  }
  return check_launch("gemm_bf16");
}
