// Grouped W8A16 GEMV plans: many independent GEMVs streamed by one launch per
// slot class from a descriptor table resolved once and kept in device memory.
//
// This is the multi-matrix form of infer::cuda::gemv_w8a16
// (include/infer/cuda_ops.hpp:47-50) for callers that issue several GEMVs on
// the same stream with no dependency between them: q/k/v on one normed
// input and gate/up on another (src/qwen2.cpp:615-626, 646-651), or a sweep
// of many layers' Linears as tools/linear_benchmark.cpp does per case.  The
// table is built at set-up time (as the reference resolves and uploads its
// weights once, src/qwen2.cpp:56-78); launching it allocates nothing.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <new>
#include <vector>

#include "linear_kernels.hpp"
#include "status.hpp"

using namespace qlin;

struct infer_hip_gemv_plan {
  W8GroupDesc* table = nullptr;  // device memory
  int count = 0;
  int blocks = 0;
  int device = 0;
  double bytes = 0.0;
};

extern "C" int infer_hip_w8a16_gemv_plan_create(const infer_hip_w8a16_gemv_desc* descs,
                                                int count, infer_hip_gemv_plan** plan_out) {
  if (!plan_out) return fail(INFER_HIP_INVALID_ARGUMENT, "gemv plan: null output pointer");
  *plan_out = nullptr;
  if (!descs || count <= 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemv plan: need at least one descriptor");
  }
  std::vector<W8GroupDesc> table;
  table.reserve(count);
  double bytes = 0.0;
  for (int i = 0; i < count; ++i) {
    const infer_hip_w8a16_gemv_desc& d = descs[i];
    if (d.group_size != 64) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "gemv plan: descriptor %d: group size must be 64",
                  i);
    }
    if (d.out_features <= 0 || d.in_features <= 0) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "gemv plan: descriptor %d: bad shape N=%d K=%d", i,
                  d.out_features, d.in_features);
    }
    if (!d.weight || !d.scales || !d.input || !d.output) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "gemv plan: descriptor %d: null pointer", i);
    }
    if (!w8a16_gemv_fast_supported(d.weight, d.input, d.in_features)) {
      return fail(INFER_HIP_INVALID_ARGUMENT,
                  "gemv plan: descriptor %d needs K %% 64 == 0 and 16-byte aligned weight and "
                  "input (K=%d)",
                  i, d.in_features);
    }
    table.push_back(W8GroupDesc{d.weight, d.scales, d.bias, d.input, d.output, d.out_features,
                                d.in_features, 0, w8a16_grouped_rows_per_block(d.in_features)});
    bytes += static_cast<double>(d.out_features) * d.in_features +
             2.0 * d.out_features * (d.in_features / 64) + 2.0 * d.in_features +
             2.0 * d.out_features + (d.bias ? 2.0 * d.out_features : 0.0);
  }
  // Longest rows first: the blocks that take longest start earliest, which
  // shortens the launch's tail.
  std::stable_sort(table.begin(), table.end(),
                   [](const W8GroupDesc& a, const W8GroupDesc& b) { return a.k > b.k; });
  long long blocks = 0;
  for (W8GroupDesc& d : table) {
    d.block_begin = static_cast<int>(blocks);
    blocks += (d.n + d.rows_per_block - 1) / d.rows_per_block;
  }
  if (blocks > 0x7FFFFFFF) return fail(INFER_HIP_INVALID_ARGUMENT, "gemv plan: too many rows");
  auto* plan = new (std::nothrow) infer_hip_gemv_plan();
  if (!plan) return fail(INFER_HIP_RUNTIME_ERROR, "gemv plan: out of host memory");
  plan->count = count;
  plan->blocks = static_cast<int>(blocks);
  plan->bytes = bytes;
  hipError_t st = hipGetDevice(&plan->device);
  if (st == hipSuccess) st = hipMalloc(&plan->table, table.size() * sizeof(W8GroupDesc));
  if (st == hipSuccess) {
    st = hipMemcpy(plan->table, table.data(), table.size() * sizeof(W8GroupDesc),
                   hipMemcpyHostToDevice);
  }
  if (st != hipSuccess) {
    if (plan->table) (void)hipFree(plan->table);
    delete plan;
    return fail(INFER_HIP_RUNTIME_ERROR, "gemv plan: %s", hipGetErrorString(st));
  }
  *plan_out = plan;
  return ok();
}

extern "C" int infer_hip_w8a16_gemv_plan_launch(const infer_hip_gemv_plan* plan,
                                                hipStream_t stream) {
  if (!plan) return fail(INFER_HIP_INVALID_ARGUMENT, "gemv plan: null plan");
  launch_w8a16_gemv_grouped(plan->table, plan->count, plan->blocks, stream);
  return check_launch("w8a16 gemv plan");
}

extern "C" double infer_hip_w8a16_gemv_plan_bytes(const infer_hip_gemv_plan* plan) {
  return plan ? plan->bytes : 0.0;
}

extern "C" int infer_hip_w8a16_gemv_plan_destroy(infer_hip_gemv_plan* plan) {
  if (!plan) return ok();
  int prev = 0;
  hipError_t st = hipGetDevice(&prev);
  if (st == hipSuccess && prev != plan->device) st = hipSetDevice(plan->device);
  if (st == hipSuccess) st = hipFree(plan->table);
  if (prev != plan->device) (void)hipSetDevice(prev);
  delete plan;
  if (st != hipSuccess) return fail(INFER_HIP_RUNTIME_ERROR, "gemv plan: %s", hipGetErrorString(st));
  return ok();
}
