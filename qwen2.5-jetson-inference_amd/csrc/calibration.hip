// Measurement aids for bench.py, built as libinfer_calib.so beside the
// Linear library and not part of its ABI: a read-only streaming kernel (the
// HBM read rate of a kernel that does nothing but read, the practical ceiling
// for the GEMV and LM-head rooflines) and an empty kernel (the fixed cost of
// one launch, the floor under every launch of the decode step).
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 16-byte non-temporal loads (as the GEMVs read weights), four in flight per
// thread, grid-stride.  The loaded words are folded into one value that is
// stored only if it equals a constant no equal-word fill produces, so the
// loads are kept and nothing is written.
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ p, size_t n16,
                                                          unsigned* sink) {
  const size_t stride = static_cast<size_t>(gridDim.x) * 256u;
  size_t i = static_cast<size_t>(blockIdx.x) * 256u + threadIdx.x;
  unsigned acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(p + i);
    const u32x4 b = __builtin_nontemporal_load(p + i + stride);
    const u32x4 c = __builtin_nontemporal_load(p + i + 2 * stride);
    const u32x4 d = __builtin_nontemporal_load(p + i + 3 * stride);
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w;
    acc ^= c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const u32x4 a = __builtin_nontemporal_load(p + i);
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

__global__ __launch_bounds__(256) void empty_kernel() {}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16) at `data` (16-byte aligned) with `blocks`
// workgroups of 256 threads.  Returns 0, 1 for an invalid argument, 2 if the
// launch failed.
int infer_calib_stream_read(const void* data, size_t bytes, unsigned* sink, int blocks,
                            hipStream_t stream) {
  if (!data || !sink || bytes == 0 || bytes % 16 != 0 ||
      (reinterpret_cast<uintptr_t>(data) & 15u) != 0 || blocks < 1 || blocks > 65536) {
    return 1;
  }
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, stream,
                     static_cast<const u32x4*>(data), bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Launches `blocks` workgroups of 256 threads that do nothing.
int infer_calib_empty(int blocks, hipStream_t stream) {
  if (blocks < 1 || blocks > 65536) return 1;
  hipLaunchKernelGGL(empty_kernel, dim3(blocks), dim3(256), 0, stream);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
