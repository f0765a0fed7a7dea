// Decode-time (M = 1) Linear kernels for gfx950: W8A16 group-64 GEMV, BF16
// GEMV, and the tied LM head with a fused FP32 argmax, plus the exact
// fallbacks for unaligned or ragged shapes.
//
// Mapping (all fast kernels).  The weight matrix is row-major [N, K], so a
// row is one contiguous run of K int8 (or 2K bytes of BF16).  A row is cut
// into 16-byte chunks; lane l of a wave owns chunks l, l + 64, l + 128, ...
// of EVERY row it visits, so the activation values those chunks multiply are
// loaded once per wave and kept in VGPRs as FP32.  A wave then walks RB rows
// at a time: one 16-byte load per (row, chunk slot) — 64 lanes read one
// contiguous 1 KiB span, fully coalesced — and the RB per-lane partial sums
// are reduced across the wave with a reduce-scatter butterfly.
//
// Reference behaviour restated (src/cuda/kernels.cu):
//   gemv_w8a16_fast_kernel 985-1041 / dot_w8a16_sixteen 953-983: FP32 sum of
//     (float)q * (float)s * (float)x over k, + bias, BF16 RNE.
//   gemv_bf16_fast_kernel 438-490: FP32 sum of w * x, + bias, BF16 RNE.
//   lm_head_bf16_kernel 492-568 + lm_head_reduce_kernel 570-603: logits and
//     a two-stage argmax with ties to the lowest index.
//   linear_w8a16_kernel 1324-1387, gemv_bf16_scalar_kernel 396-436: any K,
//     any alignment.
#include <float.h>
#include <limits.h>
#include <stdint.h>

#include <mutex>

#include "device_common.hpp"
#include "linear_kernels.hpp"
#include "status.hpp"

namespace qlin {

namespace {

constexpr int kBlock = 256;            // 4 waves
constexpr int kWavesPerBlock = kBlock / kWave;

// ---------------------------------------------------------------- W8A16 --

// The weights and scales of one slab (64 chunks of 16 int8) of R rows.
template <int R>
__device__ __forceinline__ void w8a16_load_rows(const W8GemvArgs& a, int row0, int row_end,
                                                int c, bool cv, int groups, uint4 (&w)[R],
                                                uint32_t (&s)[R]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r;
    if (cv && row < row_end) {
      w[r] = load_stream16(a.w + static_cast<size_t>(row) * a.k + 16 * c);
      s[r] = gload(a.s + static_cast<size_t>(row) * groups + (c >> 2));
    } else {
      w[r] = make_uint4(0, 0, 0, 0);
      s[r] = 0;
    }
  }
}

// Reduce the R row sums of a task across the wave and write them.
template <int R>
__device__ __forceinline__ void w8a16_finish_rows(const W8GemvArgs& a, int row0, int row_end,
                                                  float (&acc)[R], int lane) {
  wave_reduce_rows<R>(acc, lane);
  if (is_row_writer<R>(lane)) {
    const int row = row0 + reduced_row<R>(lane);
    if (row < row_end) {
      const float b = a.bias ? bf16_to_f32(gload(a.bias + row)) : 0.0f;
      gstore(a.y + row, f32_to_bf16(acc[0] + b));
    }
  }
}

// The activations of one slab chunk c (16 BF16 as FP32), zero past K.
__device__ __forceinline__ void w8a16_load_x(const W8GemvArgs& a, int c, bool cv,
                                             float (&x)[16]) {
  if (cv) {
    load_x16(a.x + 16 * c, x);
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) x[e] = 0.0f;
  }
}

// One wave's share of a W8A16 GEMV: the R-row tasks starting at rows
// first, first + stride, ... below row_end.  A row is walked in slabs of
// 64 chunks (1 KiB of int8); lane l takes chunk l of every slab, so a lane
// multiplies the same 16 activations into each of the R rows of a slab.
// Per lane the sum is acc = fma(dot16(q, x), s, acc) slab by slab.
// PF: the loads of the next (task, slab) unit are issued before the current
// unit is computed, so each wave keeps two units in flight.
// Requires K % 64 == 0, 16-byte aligned weight and input.
template <int R, bool PF>
__device__ __forceinline__ void w8a16_wave_span(const W8GemvArgs& a, int first, int stride,
                                                int row_end) {
  if (first >= row_end) return;
  const int lane = threadIdx.x & (kWave - 1);
  const int chunks = a.k >> 4;
  const int groups = a.k >> 6;
  const int slabs = (chunks + kWave - 1) / kWave;
  if (slabs == 1) {
    // K <= 1024: the activations stay in VGPRs for every task.
    const bool cv = lane < chunks;
    float x[16];
    w8a16_load_x(a, lane, cv, x);
    uint4 w[R];
    uint32_t s[R];
    w8a16_load_rows<R>(a, first, row_end, lane, cv, groups, w, s);
    for (int row0 = first; row0 < row_end; row0 += stride) {
      uint4 wn[R];
      uint32_t sn[R];
      if (PF) w8a16_load_rows<R>(a, row0 + stride, row_end, lane, cv, groups, wn, sn);
      float acc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = fmaf(dot16_i8(w[r], x), bf16_to_f32(s[r]), 0.0f);
      w8a16_finish_rows<R>(a, row0, row_end, acc, lane);
      if (PF) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          w[r] = wn[r];
          s[r] = sn[r];
        }
      } else {
        w8a16_load_rows<R>(a, row0 + stride, row_end, lane, cv, groups, w, s);
      }
    }
    return;
  }
  // K > 1024: walk (task, slab) units in order, activations per slab.
  int row0 = first;
  int slab = 0;
  float x[16];
  uint4 w[R];
  uint32_t s[R];
  w8a16_load_x(a, lane, lane < chunks, x);
  w8a16_load_rows<R>(a, row0, row_end, lane, lane < chunks, groups, w, s);
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  while (row0 < row_end) {
    const bool last = slab + 1 == slabs;
    const int nrow0 = last ? row0 + stride : row0;
    const int nslab = last ? 0 : slab + 1;
    const int nc = nslab * kWave + lane;
    const bool ncv = nc < chunks;
    float xn[16];
    uint4 wn[R];
    uint32_t sn[R];
    if (PF) {
      w8a16_load_x(a, nc, ncv && nrow0 < row_end, xn);
      w8a16_load_rows<R>(a, nrow0, row_end, nc, ncv, groups, wn, sn);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = fmaf(dot16_i8(w[r], x), bf16_to_f32(s[r]), acc[r]);
    if (last) {
      w8a16_finish_rows<R>(a, row0, row_end, acc, lane);
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    }
    if (PF) {
#pragma unroll
      for (int e = 0; e < 16; ++e) x[e] = xn[e];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        w[r] = wn[r];
        s[r] = sn[r];
      }
    } else {
      w8a16_load_x(a, nc, ncv && nrow0 < row_end, x);
      w8a16_load_rows<R>(a, nrow0, row_end, nc, ncv, groups, w, s);
    }
    row0 = nrow0;
    slab = nslab;
  }
}

// A single W8A16 GEMV: block b owns rows [b RPB, (b + 1) RPB); its waves take
// R-row tasks round-robin.
template <int R, int W, bool PF>
__global__ __launch_bounds__(kBlock, W) void w8a16_gemv_kernel(W8GemvArgs a,
                                                               int rows_per_block) {
  const int begin = blockIdx.x * rows_per_block;
  const int end = min(a.n, begin + rows_per_block);
  const int wave = threadIdx.x / kWave;
  w8a16_wave_span<R, PF>(a, begin + wave * R, kWavesPerBlock * R, end);
}

// A single W8A16 GEMV with rows longer than one slab, split over K: block b
// owns rows [b R, b R + R) and wave w takes slabs w, w + 4, ..., so all slabs
// of a row are in flight at once (a lone GEMV is latency-bound); the four
// wave partials are summed through LDS in wave order.
template <int R>
__global__ __launch_bounds__(kBlock) void w8a16_gemv_splitk_kernel(W8GemvArgs a) {
  __shared__ float part[kWavesPerBlock][R];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row0 = blockIdx.x * R;
  const int chunks = a.k >> 4;
  const int groups = a.k >> 6;
  const int slabs = (chunks + kWave - 1) / kWave;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  for (int slab = wave; slab < slabs; slab += kWavesPerBlock) {
    const int c = slab * kWave + lane;
    const bool cv = c < chunks;
    float x[16];
    w8a16_load_x(a, c, cv, x);
    uint4 w[R];
    uint32_t s[R];
    w8a16_load_rows<R>(a, row0, a.n, c, cv, groups, w, s);
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = fmaf(dot16_i8(w[r], x), bf16_to_f32(s[r]), acc[r]);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) part[wave][r] = acc[r];
  }
  __syncthreads();
  if (threadIdx.x < R) {
    const int row = row0 + threadIdx.x;
    if (row < a.n) {
      float v = part[0][threadIdx.x];
      for (int w = 1; w < kWavesPerBlock; ++w) v += part[w][threadIdx.x];
      const float b = a.bias ? bf16_to_f32(gload(a.bias + row)) : 0.0f;
      gstore(a.y + row, f32_to_bf16(v + b));
    }
  }
}

// Many W8A16 GEMVs in one launch.  Block b belongs to the descriptor d with
// block_begin[d] <= b < block_begin[d + 1] (descriptors sorted by
// block_begin) and owns rows [RPB_d (b - block_begin[d]), ...) of it.
// W = minimum waves per SIMD the register allocation must allow.
template <int R, int W, bool PF>
__global__ __launch_bounds__(kBlock, W) void w8a16_gemv_grouped_kernel(
    const W8GroupDesc* __restrict__ descs, int count) {
  const int b = blockIdx.x;
  int lo = 0, hi = count - 1;
  while (lo < hi) {  // last descriptor whose block_begin <= b
    const int mid = (lo + hi + 1) >> 1;
    if (descs[mid].block_begin <= b) lo = mid; else hi = mid - 1;
  }
  const W8GroupDesc& d = descs[lo];
  const W8GemvArgs a{d.w, d.s, d.bias, d.x, d.y, d.n, d.k};
  const int begin = (b - d.block_begin) * d.rows_per_block;
  const int end = min(d.n, begin + d.rows_per_block);
  const int wave = threadIdx.x / kWave;
  w8a16_wave_span<R, PF>(a, begin + wave * R, kWavesPerBlock * R, end);
}

// Any K, any alignment, any token count; each wave walks (token, row) items
// grid-stride.  Group index k / group_size with scale row stride
// ceil(K / group_size), as linear_w8a16_kernel (kernels.cu:1333-1339,
// 1366-1367).
__global__ __launch_bounds__(kBlock) void w8a16_linear_generic_kernel(
    const int8_t* __restrict__ w, const uint16_t* __restrict__ s, int group_size,
    const uint16_t* __restrict__ bias, const uint16_t* __restrict__ x,
    uint16_t* __restrict__ y, int tokens, int n, int k) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long items = static_cast<long long>(tokens) * n;
  const long long nwaves = static_cast<long long>(gridDim.x) * kWavesPerBlock;
  const int groups = (k + group_size - 1) / group_size;
  for (long long item = (static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x) / kWave;
       item < items; item += nwaves) {
    const int token = static_cast<int>(item / n);
    const int row = static_cast<int>(item % n);
    const int8_t* wr = w + static_cast<size_t>(row) * k;
    const uint16_t* sr = s + static_cast<size_t>(row) * groups;
    const uint16_t* xr = x + static_cast<size_t>(token) * k;
    float sum = 0.0f;
    for (int col = lane; col < k; col += kWave) {
      const float dq = static_cast<float>(wr[col]) * bf16_to_f32(sr[col / group_size]);
      sum = fmaf(dq, bf16_to_f32(xr[col]), sum);
    }
    sum = wave_sum(sum);
    if (lane == 0) {
      const float b = bias ? bf16_to_f32(bias[row]) : 0.0f;
      y[static_cast<size_t>(token) * n + row] = f32_to_bf16(sum + b);
    }
  }
}

// ----------------------------------------------------------------- BF16 --


// One wave's share of a BF16 GEMV, as w8a16_wave_span: R-row tasks, rows
// walked in slabs of 64 chunks of 8 BF16 (1 KiB); for K <= 1024 (at most
// two slabs) the activations stay in VGPRs.  Per lane the sum is a plain
// FMA chain over the lane's chunks in order.  ARGMAX also folds
// (sum + bias, row) of every written row into (best_v, best_i).
// Requires K % 8 == 0, 16-byte aligned weight and input.
template <int R, bool ARGMAX>
__device__ __forceinline__ void bf16_wave_span(const Bf16GemvArgs& a, int first, int stride,
                                               int row_end, float& best_v, int& best_i) {
  const int lane = threadIdx.x & (kWave - 1);
  const int chunks = a.k >> 3;
  const int slabs = (chunks + kWave - 1) / kWave;
  const bool hoist = slabs <= 2;
  float xh[2][8];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int c = j * kWave + lane;
    if (hoist && c < chunks) {
      load_x8(a.x + 8 * c, xh[j]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) xh[j][e] = 0.0f;
    }
  }
  for (int row0 = first; row0 < row_end; row0 += stride) {
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    if (hoist) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = j * kWave + lane;
        uint4 w[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int row = row0 + r;
          w[r] = (j < slabs && c < chunks && row < row_end)
                     ? load_stream16(a.w + static_cast<size_t>(row) * a.k + 8 * c)
                     : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = dot8_bf16(w[r], xh[j], acc[r]);
      }
    } else {
      for (int slab = 0; slab < slabs; ++slab) {
        const int c = slab * kWave + lane;
        const bool cv = c < chunks;
        float x[8];
        if (cv) {
          load_x8(a.x + 8 * c, x);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = 0.0f;
        }
        uint4 w[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int row = row0 + r;
          w[r] = (cv && row < row_end)
                     ? load_stream16(a.w + static_cast<size_t>(row) * a.k + 8 * c)
                     : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = dot8_bf16(w[r], x, acc[r]);
      }
    }
    wave_reduce_rows<R>(acc, lane);
    if (is_row_writer<R>(lane)) {
      const int row = row0 + reduced_row<R>(lane);
      if (row < row_end) {
        const float v = acc[0] + (a.bias ? bf16_to_f32(gload(a.bias + row)) : 0.0f);
        gstore(a.y + row, f32_to_bf16(v));
        if (ARGMAX && better(v, row, best_v, best_i)) {
          best_v = v;
          best_i = row;
        }
      }
    }
  }
}

// Fold (best_v, best_i) of every lane of the block into one pair per block.
__device__ __forceinline__ void block_argmax_store(float best_v, int best_i,
                                                   float* __restrict__ block_value,
                                                   int* __restrict__ block_index) {
  __shared__ float sv[kWavesPerBlock];
  __shared__ int si[kWavesPerBlock];
  const int lane = threadIdx.x & (kWave - 1);
  wave_argmax(best_v, best_i);
  const int wave_in_block = threadIdx.x / kWave;
  if (lane == 0) {
    sv[wave_in_block] = best_v;
    si[wave_in_block] = best_i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = sv[0];
    int i = si[0];
    for (int w = 1; w < kWavesPerBlock; ++w) {
      if (better(sv[w], si[w], v, i)) {
        v = sv[w];
        i = si[w];
      }
    }
    block_value[blockIdx.x] = v;
    block_index[blockIdx.x] = i;
  }
}

// A single BF16 GEMV (ARGMAX: the LM head's first stage).  Block b owns rows
// [b RPB, (b + 1) RPB).
template <int R, int W, bool ARGMAX>
__global__ __launch_bounds__(kBlock, W) void bf16_gemv_kernel(
    Bf16GemvArgs a, int rows_per_block, float* __restrict__ block_value,
    int* __restrict__ block_index) {
  const int begin = blockIdx.x * rows_per_block;
  const int end = min(a.n, begin + rows_per_block);
  const int wave = threadIdx.x / kWave;
  float best_v = -INFINITY;
  int best_i = INT_MAX;
  bf16_wave_span<R, ARGMAX>(a, begin + wave * R, kWavesPerBlock * R, end, best_v, best_i);
  if (ARGMAX) block_argmax_store(best_v, best_i, block_value, block_index);
}

// A single BF16 GEMV with rows of more than two slabs, split over K as
// w8a16_gemv_splitk_kernel: block b owns rows [b R, b R + R), wave w takes
// slabs w, w + 4, ..., partials summed through LDS in wave order.
template <int R>
__global__ __launch_bounds__(kBlock) void bf16_gemv_splitk_kernel(Bf16GemvArgs a) {
  __shared__ float part[kWavesPerBlock][R];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int row0 = blockIdx.x * R;
  const int chunks = a.k >> 3;
  const int slabs = (chunks + kWave - 1) / kWave;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  for (int slab = wave; slab < slabs; slab += kWavesPerBlock) {
    const int c = slab * kWave + lane;
    const bool cv = c < chunks;
    float x[8];
    if (cv) {
      load_x8(a.x + 8 * c, x);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = 0.0f;
    }
    uint4 w[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
      w[r] = (cv && row < a.n) ? load_stream16(a.w + static_cast<size_t>(row) * a.k + 8 * c)
                              : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = dot8_bf16(w[r], x, acc[r]);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) part[wave][r] = acc[r];
  }
  __syncthreads();
  if (threadIdx.x < R) {
    const int row = row0 + threadIdx.x;
    if (row < a.n) {
      float v = part[0][threadIdx.x];
      for (int w = 1; w < kWavesPerBlock; ++w) v += part[w][threadIdx.x];
      const float b = a.bias ? bf16_to_f32(gload(a.bias + row)) : 0.0f;
      gstore(a.y + row, f32_to_bf16(v + b));
    }
  }
}

// Second argmax stage: one block of 1024 threads folds the per-block
// winners, kReduceBatch independent loads in flight per thread (the LM head
// of V = 151936 has 9,496 winners: one round of loads instead of three with
// four; the comparison is a total order, so the order of folding does not
// change the result).  A block whose rows were all NaN reports INT_MAX; if
// every block does, the result is 0, which is what std::max_element returns
// for an all-NaN range.
constexpr int kReduceThreads = 1024;
constexpr int kReduceBatch = 16;

__global__ __launch_bounds__(kReduceThreads) void argmax_reduce_kernel(
    const float* __restrict__ block_value, const int* __restrict__ block_index,
    int count, int* __restrict__ argmax) {
  float v = -INFINITY;
  int i = INT_MAX;
  for (int b = threadIdx.x; b < count; b += kReduceBatch * kReduceThreads) {
    float cv[kReduceBatch];
    int ci[kReduceBatch];
#pragma unroll
    for (int u = 0; u < kReduceBatch; ++u) {
      const int at = b + u * kReduceThreads;
      cv[u] = at < count ? block_value[at] : -INFINITY;
      ci[u] = at < count ? block_index[at] : INT_MAX;
    }
#pragma unroll
    for (int u = 0; u < kReduceBatch; ++u) {
      if (better(cv[u], ci[u], v, i)) {
        v = cv[u];
        i = ci[u];
      }
    }
  }
  constexpr int kWaves = kReduceThreads / kWave;
  __shared__ float sv[kWaves];
  __shared__ int si[kWaves];
  wave_argmax(v, i);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  if (lane == 0) {
    sv[wave] = v;
    si[wave] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    v = sv[0];
    i = si[0];
    for (int w = 1; w < kWaves; ++w) {
      if (better(sv[w], si[w], v, i)) {
        v = sv[w];
        i = si[w];
      }
    }
    *argmax = (i == INT_MAX) ? 0 : i;
  }
}

// Any K, any alignment, any token count; each wave walks (token, row) items
// grid-stride.  ARGMAX additionally folds (sum + bias, row) to one winner per
// block (used with tokens == 1 only).
template <bool ARGMAX>
__global__ __launch_bounds__(kBlock) void bf16_linear_generic_kernel(
    const uint16_t* __restrict__ w, const uint16_t* __restrict__ bias,
    const uint16_t* __restrict__ x, uint16_t* __restrict__ y, int tokens, int n,
    int k, float* __restrict__ block_value, int* __restrict__ block_index) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long items = static_cast<long long>(tokens) * n;
  const long long nwaves = static_cast<long long>(gridDim.x) * kWavesPerBlock;
  float best_v = -INFINITY;
  int best_i = INT_MAX;
  for (long long item = (static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x) / kWave;
       item < items; item += nwaves) {
    const int token = static_cast<int>(item / n);
    const int row = static_cast<int>(item % n);
    const uint16_t* wr = w + static_cast<size_t>(row) * k;
    const uint16_t* xr = x + static_cast<size_t>(token) * k;
    float sum = 0.0f;
    for (int col = lane; col < k; col += kWave) {
      sum = fmaf(bf16_to_f32(wr[col]), bf16_to_f32(xr[col]), sum);
    }
    sum = wave_sum(sum);
    const float v = sum + (bias ? bf16_to_f32(bias[row]) : 0.0f);
    if (lane == 0) y[static_cast<size_t>(token) * n + row] = f32_to_bf16(v);
    if (ARGMAX && better(v, row, best_v, best_i)) {
      best_v = v;
      best_i = row;
    }
  }
  if (ARGMAX) {
    __shared__ float sv[kWavesPerBlock];
    __shared__ int si[kWavesPerBlock];
    const int wave_in_block = threadIdx.x / kWave;
    if (lane == 0) {
      sv[wave_in_block] = best_v;
      si[wave_in_block] = best_i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float v = sv[0];
      int i = si[0];
      for (int wv = 1; wv < kWavesPerBlock; ++wv) {
        if (better(sv[wv], si[wv], v, i)) {
          v = sv[wv];
          i = si[wv];
        }
      }
      block_value[blockIdx.x] = v;
      block_index[blockIdx.x] = i;
    }
  }
}

// ------------------------------------------------------------ dispatch --

bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// The argmax variant keeps its grid at or below ceil(N / 8) blocks so that
// its per-block scratch never exceeds the reference's LM-head workspace
// sizing (src/qwen2.cpp:193-198).
int argmax_block_cap(int n) { return (n + 7) / 8; }

// Launch geometry of a single GEMV: R rows per wave task, RPB rows per block.
// Small N is latency-bound, so it is spread over as many blocks as possible
// (4 rows per block); large N streams 2-row tasks, two per wave (the LM-head
// sweep's best: 6.76 TB/s at N = 151936).  The argmax variant needs at least
// 8 rows per block.
struct Geometry {
  int r;
  int rows_per_block;
  int blocks;
};

Geometry single_geometry(int n, bool argmax) {
  int r = 1, t = 1;
  if (n >= 65536) {
    r = 2;
    t = 2;
  } else if (n >= 4096 || argmax) {
    r = 2;
  }
  const int rpb = kWavesPerBlock * r * t;
  return {r, rpb, (n + rpb - 1) / rpb};
}

template <int R>
void launch_w8(const W8GemvArgs& a, const Geometry& g, hipStream_t stream) {
  hipLaunchKernelGGL((w8a16_gemv_kernel<R, 1, true>), dim3(g.blocks), dim3(kBlock), 0, stream,
                     a, g.rows_per_block);
}

template <int R, bool ARGMAX>
void launch_bf16(const Bf16GemvArgs& a, const Geometry& g, float* bv, int* bi,
                 hipStream_t stream) {
  hipLaunchKernelGGL((bf16_gemv_kernel<R, 6, ARGMAX>), dim3(g.blocks), dim3(kBlock), 0, stream,
                     a, g.rows_per_block, bv, bi);
}

template <bool ARGMAX>
int dispatch_bf16(const Bf16GemvArgs& a, float* bv, int* bi, hipStream_t stream) {
  const int slabs = (a.k / 8 + kWave - 1) / kWave;
  if (!ARGMAX && slabs > 2 && a.n < 65536) {
    // Long rows, few of them: split K across the waves of a block.
    if (a.n >= 2048) {
      hipLaunchKernelGGL((bf16_gemv_splitk_kernel<2>), dim3((a.n + 1) / 2), dim3(kBlock), 0,
                         stream, a);
    } else {
      hipLaunchKernelGGL((bf16_gemv_splitk_kernel<1>), dim3(a.n), dim3(kBlock), 0, stream, a);
    }
    return 0;
  }
  const Geometry g = single_geometry(a.n, ARGMAX);
  if (g.r == 1) {
    launch_bf16<1, ARGMAX>(a, g, bv, bi, stream);
  } else {
    launch_bf16<2, ARGMAX>(a, g, bv, bi, stream);
  }
  return g.blocks;
}

// Slab loops take any K; the bound keeps K in int range arithmetic.
constexpr int kMaxFastK = 1 << 20;

bool bf16_fast_ok(const uint16_t* w, const uint16_t* x, int k) {
  return k >= 8 && (k & 7) == 0 && k <= kMaxFastK && aligned16(w) && aligned16(x);
}

bool w8_fast_ok(const int8_t* w, const uint16_t* x, int k) {
  return k >= 64 && (k & 63) == 0 && k <= kMaxFastK && aligned16(w) && aligned16(x);
}

int generic_blocks(int tokens, int n) {
  const long long waves = static_cast<long long>(tokens) * n;
  const long long blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  return static_cast<int>(blocks < 65536 ? blocks : 65536);
}

// Grouped kernel: 4-row wave tasks, registers capped for >= 4 waves per
// SIMD, no register prefetch — the best of a sweep over R in {2, 4, 8},
// waves per SIMD in {1, 4, 6, 8}, prefetch on/off and tasks per wave on the
// 168-GEMV decode set (6.58 TB/s against 6.80 TB/s for a bare streaming
// read of the same 370 MB).
constexpr int kGroupedR = 4;
constexpr int kGroupedWaves = 4;
constexpr bool kGroupedPrefetch = false;

}  // namespace

// ------------------------------------------------------ internal entries --

void launch_w8a16_gemv_fast(const W8GemvArgs& a, hipStream_t stream) {
  const int slabs = (a.k / 16 + kWave - 1) / kWave;
  if (slabs > 1 && a.n < 65536) {
    // Long rows, few of them: split K across the waves of a block.
    if (a.n >= 2048) {
      hipLaunchKernelGGL((w8a16_gemv_splitk_kernel<2>), dim3((a.n + 1) / 2), dim3(kBlock), 0,
                         stream, a);
    } else {
      hipLaunchKernelGGL((w8a16_gemv_splitk_kernel<1>), dim3(a.n), dim3(kBlock), 0, stream, a);
    }
    return;
  }
  const Geometry g = single_geometry(a.n, false);
  if (g.r == 1) {
    launch_w8<1>(a, g, stream);
  } else {
    launch_w8<2>(a, g, stream);
  }
}

bool w8a16_gemv_fast_supported(const int8_t* w, const uint16_t* x, int k) {
  return w8_fast_ok(w, x, k);
}

int w8a16_grouped_rows_per_block(int k) {
  // Four tasks per wave for K <= 1024 (one slab), two for longer rows.
  const int slabs = (k / 16 + kWave - 1) / kWave;
  return kWavesPerBlock * kGroupedR * (slabs == 1 ? 4 : 2);
}

void launch_w8a16_gemv_grouped(const W8GroupDesc* descs, int count, int total_blocks,
                               hipStream_t stream) {
  hipLaunchKernelGGL((w8a16_gemv_grouped_kernel<kGroupedR, kGroupedWaves, kGroupedPrefetch>),
                     dim3(total_blocks), dim3(kBlock),
                     0, stream, descs, count);
}

void launch_w8a16_linear_generic(const int8_t* w, const uint16_t* s, int group_size,
                                 const uint16_t* bias, const uint16_t* x, uint16_t* y,
                                 int tokens, int n, int k, hipStream_t stream) {
  hipLaunchKernelGGL(w8a16_linear_generic_kernel, dim3(generic_blocks(tokens, n)), dim3(kBlock),
                     0, stream, w, s, group_size, bias, x, y, tokens, n, k);
}

void launch_bf16_linear_generic(const uint16_t* w, const uint16_t* bias, const uint16_t* x,
                                uint16_t* y, int tokens, int n, int k, hipStream_t stream) {
  hipLaunchKernelGGL(bf16_linear_generic_kernel<false>, dim3(generic_blocks(tokens, n)),
                     dim3(kBlock), 0, stream, w, bias, x, y, tokens, n, k, nullptr, nullptr);
}

bool bf16_gemv_fast_supported(const uint16_t* w, const uint16_t* x, int k) {
  return bf16_fast_ok(w, x, k);
}

void launch_bf16_gemv_fast(const Bf16GemvArgs& a, hipStream_t stream) {
  dispatch_bf16<false>(a, nullptr, nullptr, stream);
}

// Blocks the LM head's first stage uses (its workspace entry count).
size_t lm_head_blocks(int vocab, int in_features, bool fast) {
  if (vocab <= 0 || in_features < 0) return 0;
  int blocks = fast ? single_geometry(vocab, true).blocks : generic_blocks(1, vocab);
  const int cap = argmax_block_cap(vocab);
  return static_cast<size_t>(blocks < cap ? blocks : cap);
}

}  // namespace qlin

// ================================================================ C ABI ==

using namespace qlin;

extern "C" int infer_hip_gemv_w8a16(const int8_t* weight, const uint16_t* scales,
                                    int group_size, const uint16_t* bias,
                                    const uint16_t* input, uint16_t* output,
                                    int out_features, int in_features, hipStream_t stream) {
  // kernels.cu:1631 — the only supported group size.
  if (group_size != 64) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "w8a16 group size must be 64 (got %d)", group_size);
  }
  if (out_features <= 0 || in_features < 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemv_w8a16: bad shape N=%d K=%d", out_features,
                in_features);
  }
  if (!output || (in_features > 0 && (!weight || !scales || !input))) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemv_w8a16: null required pointer");
  }
  if (w8_fast_ok(weight, input, in_features)) {
    launch_w8a16_gemv_fast({weight, scales, bias, input, output, out_features, in_features},
                           stream);
  } else {
    launch_w8a16_linear_generic(weight, scales, group_size, bias, input, output, 1, out_features,
                                in_features, stream);
  }
  return check_launch("gemv_w8a16");
}

extern "C" int infer_hip_gemv_bf16(const uint16_t* weight, const uint16_t* bias,
                                   const uint16_t* input, uint16_t* output, int out_features,
                                   int in_features, hipStream_t stream) {
  if (out_features <= 0 || in_features < 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemv_bf16: bad shape N=%d K=%d", out_features,
                in_features);
  }
  if (!output || (in_features > 0 && (!weight || !input))) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemv_bf16: null required pointer");
  }
  if (bf16_fast_ok(weight, input, in_features)) {
    launch_bf16_gemv_fast({weight, bias, input, output, out_features, in_features}, stream);
  } else {
    launch_bf16_linear_generic(weight, bias, input, output, 1, out_features, in_features, stream);
  }
  return check_launch("gemv_bf16");
}

extern "C" size_t infer_hip_lm_head_workspace_entries(int vocab, int in_features) {
  // The fast path (aligned pointers) uses the larger of the two counts only
  // when it is the generic one, so report the maximum of both.
  const size_t fast = lm_head_blocks(vocab, in_features, true);
  const size_t slow = lm_head_blocks(vocab, in_features, false);
  return fast > slow ? fast : slow;
}

namespace {

// The LM head after argument checks: the first stage (logits and one
// (value, index) winner per block into block_max_value / block_max_index),
// then the single-block argmax over those winners.
int launch_lm_head(const uint16_t* weight, const uint16_t* bias, const uint16_t* input,
                   uint16_t* logits, float* block_max_value, int* block_max_index, int* argmax,
                   int vocab, int in_features, hipStream_t stream) {
  int blocks;
  if (bf16_fast_ok(weight, input, in_features)) {
    blocks = dispatch_bf16<true>({weight, bias, input, logits, vocab, in_features},
                                 block_max_value, block_max_index, stream);
  } else {
    blocks = generic_blocks(1, vocab);
    if (blocks > argmax_block_cap(vocab)) blocks = argmax_block_cap(vocab);
    hipLaunchKernelGGL(bf16_linear_generic_kernel<true>, dim3(blocks), dim3(kBlock), 0, stream,
                       weight, bias, input, logits, 1, vocab, in_features, block_max_value,
                       block_max_index);
  }
  int rc = check_launch("lm_head_bf16");
  if (rc != INFER_HIP_OK) return rc;
  hipLaunchKernelGGL(argmax_reduce_kernel, dim3(1), dim3(kReduceThreads), 0, stream,
                     block_max_value, block_max_index, blocks, argmax);
  return check_launch("lm_head_bf16 argmax");
}

int check_lm_head_args(const uint16_t* weight, const uint16_t* input, const uint16_t* logits,
                       const int* argmax, int vocab, int in_features, const char* what) {
  if (vocab <= 0 || in_features < 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: bad shape V=%d K=%d", what, vocab,
                in_features);
  }
  if (!logits || !argmax || (in_features > 0 && (!weight || !input))) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null required pointer", what);
  }
  return INFER_HIP_OK;
}

// ------------------------------------------- static scratch (no allocation) --
//
// The winners of infer_hip_lm_head_bf16_noalloc's first stage live in this
// file-scope device array instead of a caller workspace: kNoAllocEntries
// (value, index) pairs, values in the first half and indices in the second,
// 512 KiB per GPU, held until the process ends.  Every call on one GPU uses
// that GPU's copy; each call writes every entry it then reads, so nothing
// needs clearing between calls, and calls that overlap on one GPU race.
// 65536 entries hold the first stage of every vocab <= 2^20: at most one
// block per 16 rows (fast path, vocab >= 65536) or 65536 blocks (generic).
constexpr int kNoAllocEntries = 65536;
static __device__ __align__(256) uint32_t scratch[2 * kNoAllocEntries];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once per
// device with that device current (each GPU holds its own copy at its own
// address; in host code the array's name is only a stand-in for it).
int scratch_for_current_device(void** out) {
  int device = 0;
  hipError_t st = hipGetDevice(&device);
  if (st != hipSuccess) {
    return fail(INFER_HIP_RUNTIME_ERROR, "lm_head_bf16_noalloc: %s", hipGetErrorString(st));
  }
  if (device < 0 || device >= kMaxDevices) {
    return fail(INFER_HIP_RUNTIME_ERROR, "lm_head_bf16_noalloc: device %d beyond %d", device,
                kMaxDevices);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[device]) {
    void* ptr = nullptr;
    st = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (st != hipSuccess || !ptr) {
      return fail(INFER_HIP_RUNTIME_ERROR, "lm_head_bf16_noalloc: scratch address: %s",
                  hipGetErrorString(st));
    }
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return INFER_HIP_OK;
}

}  // namespace

extern "C" int infer_hip_lm_head_bf16(const uint16_t* weight, const uint16_t* bias,
                                      const uint16_t* input, uint16_t* logits,
                                      float* block_max_value, int* block_max_index, int* argmax,
                                      int vocab, int in_features, hipStream_t stream) {
  int rc = check_lm_head_args(weight, input, logits, argmax, vocab, in_features, "lm_head_bf16");
  if (rc != INFER_HIP_OK) return rc;
  if (!block_max_value || !block_max_index) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "lm_head_bf16: null required pointer");
  }
  return launch_lm_head(weight, bias, input, logits, block_max_value, block_max_index, argmax,
                        vocab, in_features, stream);
}

extern "C" int infer_hip_lm_head_bf16_noalloc(const uint16_t* weight, const uint16_t* bias,
                                              const uint16_t* input, uint16_t* logits,
                                              int* argmax, int vocab, int in_features,
                                              hipStream_t stream) {
  const char* what = "lm_head_bf16_noalloc";
  int rc = check_lm_head_args(weight, input, logits, argmax, vocab, in_features, what);
  if (rc != INFER_HIP_OK) return rc;
  const size_t entries = infer_hip_lm_head_workspace_entries(vocab, in_features);
  if (entries > static_cast<size_t>(kNoAllocEntries)) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "%s: V=%d needs %zu scratch entries, more than the static %d (V <= %d)", what,
                vocab, entries, kNoAllocEntries, 16 * kNoAllocEntries);
  }
  void* ptr = nullptr;
  rc = scratch_for_current_device(&ptr);
  if (rc != INFER_HIP_OK) return rc;
  float* values = static_cast<float*>(ptr);
  int* indices = static_cast<int*>(ptr) + kNoAllocEntries;
  return launch_lm_head(weight, bias, input, logits, values, indices, argmax, vocab, in_features,
                        stream);
}
