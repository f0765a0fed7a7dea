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

#include "device_common.hpp"
#include "linear_kernels.hpp"
#include "status.hpp"

namespace qlin {

namespace {

constexpr int kBlock = 256;            // 4 waves
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kMaxWaves = 256 * 16;    // persistent cap: 16 waves per CU

// ---------------------------------------------------------------- W8A16 --

// Dot product of one 16-byte chunk of int8 weights with 16 FP32 activations.
__device__ __forceinline__ float dot16_i8(const uint4 w, const float (&x)[16]) {
  float p = sbyte0(w.x) * x[0];
  p = fmaf(sbyte1(w.x), x[1], p);
  p = fmaf(sbyte2(w.x), x[2], p);
  p = fmaf(sbyte3(w.x), x[3], p);
  p = fmaf(sbyte0(w.y), x[4], p);
  p = fmaf(sbyte1(w.y), x[5], p);
  p = fmaf(sbyte2(w.y), x[6], p);
  p = fmaf(sbyte3(w.y), x[7], p);
  p = fmaf(sbyte0(w.z), x[8], p);
  p = fmaf(sbyte1(w.z), x[9], p);
  p = fmaf(sbyte2(w.z), x[10], p);
  p = fmaf(sbyte3(w.z), x[11], p);
  p = fmaf(sbyte0(w.w), x[12], p);
  p = fmaf(sbyte1(w.w), x[13], p);
  p = fmaf(sbyte2(w.w), x[14], p);
  p = fmaf(sbyte3(w.w), x[15], p);
  return p;
}

// Load 16 BF16 activations (32 bytes) as FP32.
__device__ __forceinline__ void load_x16(const uint16_t* x, float (&out)[16]) {
  const uint4 a = *reinterpret_cast<const uint4*>(x);
  const uint4 b = *reinterpret_cast<const uint4*>(x + 8);
  out[0] = bf16_lo(a.x);  out[1] = bf16_hi(a.x);
  out[2] = bf16_lo(a.y);  out[3] = bf16_hi(a.y);
  out[4] = bf16_lo(a.z);  out[5] = bf16_hi(a.z);
  out[6] = bf16_lo(a.w);  out[7] = bf16_hi(a.w);
  out[8] = bf16_lo(b.x);  out[9] = bf16_hi(b.x);
  out[10] = bf16_lo(b.y); out[11] = bf16_hi(b.y);
  out[12] = bf16_lo(b.z); out[13] = bf16_hi(b.z);
  out[14] = bf16_lo(b.w); out[15] = bf16_hi(b.w);
}

// One wave's share of a W8A16 GEMV: row steps first, first + stride, ...
// below end, RB rows per step.  S = chunk slots per lane (K <= 1024 S).
// Requires K % 64 == 0, 16-byte aligned weight and input.
template <int S, int RB>
__device__ __forceinline__ void w8a16_wave_rows(const W8GemvArgs& a, int first, int stride,
                                                int end) {
  const int lane = threadIdx.x & (kWave - 1);
  const int chunks = a.k >> 4;
  const int groups = a.k >> 6;

  float xr[S][16];
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const int c = lane + kWave * j;
    if (c < chunks) {
      load_x16(a.x + 16 * c, xr[j]);
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) xr[j][e] = 0.0f;
    }
  }

  for (int step = first; step < end; step += stride) {
    const int r0 = step * RB;
    uint4 wv[RB][S];
    uint32_t sv[RB][S];
#pragma unroll
    for (int rr = 0; rr < RB; ++rr) {
      const int row = r0 + rr;
#pragma unroll
      for (int j = 0; j < S; ++j) {
        const int c = lane + kWave * j;
        if (row < a.n && c < chunks) {
          wv[rr][j] = load_stream16(a.w + static_cast<size_t>(row) * a.k + 16 * c);
          sv[rr][j] = a.s[static_cast<size_t>(row) * groups + (c >> 2)];
        } else {
          wv[rr][j] = make_uint4(0, 0, 0, 0);
          sv[rr][j] = 0;
        }
      }
    }
    float acc[RB];
#pragma unroll
    for (int rr = 0; rr < RB; ++rr) {
      acc[rr] = 0.0f;
#pragma unroll
      for (int j = 0; j < S; ++j) {
        acc[rr] = fmaf(dot16_i8(wv[rr][j], xr[j]), bf16_to_f32(sv[rr][j]), acc[rr]);
      }
    }
    wave_reduce_rows<RB>(acc, lane);
    if (is_row_writer<RB>(lane)) {
      const int row = r0 + reduced_row<RB>(lane);
      if (row < a.n) {
        const float b = a.bias ? bf16_to_f32(a.bias[row]) : 0.0f;
        a.y[row] = f32_to_bf16(acc[0] + b);
      }
    }
  }
}

// A single W8A16 GEMV; waves walk row steps grid-stride.
template <int S, int RB>
__global__ __launch_bounds__(kBlock) void w8a16_gemv_kernel(W8GemvArgs a) {
  const int wave = (blockIdx.x * kBlock + threadIdx.x) / kWave;
  const int nwaves = gridDim.x * kWavesPerBlock;
  w8a16_wave_rows<S, RB>(a, wave, nwaves, (a.n + RB - 1) / RB);
}

// Many W8A16 GEMVs of one slot class S in one launch.  Block b belongs to
// the descriptor d with block_begin[d] <= b < block_begin[d + 1] (descriptors
// sorted by block_begin); within it, block b - block_begin[d] owns rows
// [RPB (b - begin), RPB (b - begin + 1)), RPB = kWavesPerBlock * RB * kSteps.
template <int S, int RB, int kSteps>
__global__ __launch_bounds__(kBlock) void w8a16_gemv_grouped_kernel(
    const W8GroupDesc* __restrict__ descs, int count) {
  constexpr int kRowsPerBlock = kWavesPerBlock * RB * kSteps;
  const int b = blockIdx.x;
  int lo = 0, hi = count - 1;
  while (lo < hi) {  // last descriptor whose block_begin <= b
    const int mid = (lo + hi + 1) >> 1;
    if (descs[mid].block_begin <= b) lo = mid; else hi = mid - 1;
  }
  const W8GroupDesc& d = descs[lo];
  const W8GemvArgs a{d.w, d.s, d.bias, d.x, d.y, d.n, d.k};
  const int local = b - d.block_begin;
  const int wave = threadIdx.x / kWave;
  const int step0 = local * (kRowsPerBlock / RB);
  const int steps_total = (a.n + RB - 1) / RB;
  const int step_end = min(steps_total, step0 + kRowsPerBlock / RB);
  w8a16_wave_rows<S, RB>(a, step0 + wave, kWavesPerBlock, step_end);
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

__device__ __forceinline__ void load_x8(const uint16_t* x, float (&out)[8]) {
  const uint4 a = *reinterpret_cast<const uint4*>(x);
  out[0] = bf16_lo(a.x); out[1] = bf16_hi(a.x);
  out[2] = bf16_lo(a.y); out[3] = bf16_hi(a.y);
  out[4] = bf16_lo(a.z); out[5] = bf16_hi(a.z);
  out[6] = bf16_lo(a.w); out[7] = bf16_hi(a.w);
}

__device__ __forceinline__ float dot8_bf16(const uint4 w, const float (&x)[8], float acc) {
  acc = fmaf(bf16_lo(w.x), x[0], acc);
  acc = fmaf(bf16_hi(w.x), x[1], acc);
  acc = fmaf(bf16_lo(w.y), x[2], acc);
  acc = fmaf(bf16_hi(w.y), x[3], acc);
  acc = fmaf(bf16_lo(w.z), x[4], acc);
  acc = fmaf(bf16_hi(w.z), x[5], acc);
  acc = fmaf(bf16_lo(w.w), x[6], acc);
  acc = fmaf(bf16_hi(w.w), x[7], acc);
  return acc;
}

// Better (value, index) pair: larger value, ties to the lower index.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    const float ov = __shfl_xor(v, offset);
    const int oi = __shfl_xor(i, offset);
    if (better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

// S = 8-element chunk slots per lane (K <= 512 S), RB = rows per wave step.
// ARGMAX: also reduce the FP32 (sum + bias) of every row to one
// (value, index) per block.  Requires K % 8 == 0, 16-byte aligned weight and
// input.
template <int S, int RB, bool ARGMAX>
__global__ __launch_bounds__(kBlock) void bf16_gemv_kernel(
    Bf16GemvArgs a, float* __restrict__ block_value, int* __restrict__ block_index) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = (blockIdx.x * kBlock + threadIdx.x) / kWave;
  const int nwaves = gridDim.x * kWavesPerBlock;
  const int chunks = a.k >> 3;

  float xr[S][8];
#pragma unroll
  for (int j = 0; j < S; ++j) {
    const int c = lane + kWave * j;
    if (c < chunks) {
      load_x8(a.x + 8 * c, xr[j]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) xr[j][e] = 0.0f;
    }
  }

  float best_v = -INFINITY;
  int best_i = INT_MAX;
  const int row_steps = (a.n + RB - 1) / RB;
  for (int step = wave; step < row_steps; step += nwaves) {
    const int r0 = step * RB;
    uint4 wv[RB][S];
#pragma unroll
    for (int rr = 0; rr < RB; ++rr) {
      const int row = r0 + rr;
#pragma unroll
      for (int j = 0; j < S; ++j) {
        const int c = lane + kWave * j;
        if (row < a.n && c < chunks) {
          wv[rr][j] = load_stream16(a.w + static_cast<size_t>(row) * a.k + 8 * c);
        } else {
          wv[rr][j] = make_uint4(0, 0, 0, 0);
        }
      }
    }
    float acc[RB];
#pragma unroll
    for (int rr = 0; rr < RB; ++rr) {
      acc[rr] = 0.0f;
#pragma unroll
      for (int j = 0; j < S; ++j) acc[rr] = dot8_bf16(wv[rr][j], xr[j], acc[rr]);
    }
    wave_reduce_rows<RB>(acc, lane);
    if (is_row_writer<RB>(lane)) {
      const int row = r0 + reduced_row<RB>(lane);
      if (row < a.n) {
        const float v = acc[0] + (a.bias ? bf16_to_f32(a.bias[row]) : 0.0f);
        a.y[row] = f32_to_bf16(v);
        if (ARGMAX && better(v, row, best_v, best_i)) {
          best_v = v;
          best_i = row;
        }
      }
    }
  }

  if (ARGMAX) {
    __shared__ float sv[kWavesPerBlock];
    __shared__ int si[kWavesPerBlock];
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
}

// Second argmax stage: one block folds the per-block winners.  A block whose
// rows were all NaN reports INT_MAX; if every block does, the result is 0,
// which is what std::max_element returns for an all-NaN range.
__global__ __launch_bounds__(kBlock) void argmax_reduce_kernel(
    const float* __restrict__ block_value, const int* __restrict__ block_index,
    int count, int* __restrict__ argmax) {
  float v = -INFINITY;
  int i = INT_MAX;
  for (int b = threadIdx.x; b < count; b += kBlock) {
    if (better(block_value[b], block_index[b], v, i)) {
      v = block_value[b];
      i = block_index[b];
    }
  }
  __shared__ float sv[kWavesPerBlock];
  __shared__ int si[kWavesPerBlock];
  wave_argmax(v, i);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave_in_block = threadIdx.x / kWave;
  if (lane == 0) {
    sv[wave_in_block] = v;
    si[wave_in_block] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    v = sv[0];
    i = si[0];
    for (int w = 1; w < kWavesPerBlock; ++w) {
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

int grid_for(int row_steps) {
  const int waves = row_steps < kMaxWaves ? row_steps : kMaxWaves;
  return (waves + kWavesPerBlock - 1) / kWavesPerBlock;
}

template <int S, int RB>
void launch_w8(const W8GemvArgs& a, hipStream_t stream) {
  const int steps = (a.n + RB - 1) / RB;
  hipLaunchKernelGGL((w8a16_gemv_kernel<S, RB>), dim3(grid_for(steps)), dim3(kBlock), 0,
                     stream, a);
}

template <int S>
void launch_w8_rows(const W8GemvArgs& a, hipStream_t stream) {
  // Few rows: one row per wave step spreads them over the most CUs.
  if (S <= 2 && a.n >= 2048) {
    launch_w8<S, 4>(a, stream);
  } else if (S <= 4 && a.n >= 1024) {
    launch_w8<S, 2>(a, stream);
  } else {
    launch_w8<S, 1>(a, stream);
  }
}

// The argmax variant caps its grid at ceil(N / 8) blocks so that its
// per-block scratch never exceeds the reference's LM-head workspace sizing
// (src/qwen2.cpp:193-198); the kernels walk rows grid-stride, so any grid
// size is correct.
int argmax_block_cap(int n) { return (n + 7) / 8; }

template <int S, int RB, bool ARGMAX>
int launch_bf16(const Bf16GemvArgs& a, float* bv, int* bi, hipStream_t stream) {
  const int steps = (a.n + RB - 1) / RB;
  int blocks = grid_for(steps);
  if (ARGMAX && blocks > argmax_block_cap(a.n)) blocks = argmax_block_cap(a.n);
  hipLaunchKernelGGL((bf16_gemv_kernel<S, RB, ARGMAX>), dim3(blocks), dim3(kBlock), 0, stream,
                     a, bv, bi);
  return blocks;
}

template <int S, bool ARGMAX>
int launch_bf16_rows(const Bf16GemvArgs& a, float* bv, int* bi, hipStream_t stream) {
  if (S <= 4 && a.n >= 2048) return launch_bf16<S, 4, ARGMAX>(a, bv, bi, stream);
  if (S <= 8 && a.n >= 1024) return launch_bf16<S, 2, ARGMAX>(a, bv, bi, stream);
  return launch_bf16<S, 1, ARGMAX>(a, bv, bi, stream);
}

template <bool ARGMAX>
int dispatch_bf16(const Bf16GemvArgs& a, float* bv, int* bi, hipStream_t stream) {
  switch ((a.k + 511) / 512) {
    case 1: return launch_bf16_rows<1, ARGMAX>(a, bv, bi, stream);
    case 2: return launch_bf16_rows<2, ARGMAX>(a, bv, bi, stream);
    case 3: return launch_bf16_rows<3, ARGMAX>(a, bv, bi, stream);
    case 4: return launch_bf16_rows<4, ARGMAX>(a, bv, bi, stream);
    case 5: return launch_bf16_rows<5, ARGMAX>(a, bv, bi, stream);
    case 6: return launch_bf16_rows<6, ARGMAX>(a, bv, bi, stream);
    case 7: return launch_bf16_rows<7, ARGMAX>(a, bv, bi, stream);
    case 8: return launch_bf16_rows<8, ARGMAX>(a, bv, bi, stream);
    case 9: return launch_bf16_rows<9, ARGMAX>(a, bv, bi, stream);
    case 10: return launch_bf16_rows<10, ARGMAX>(a, bv, bi, stream);
    case 11: return launch_bf16_rows<11, ARGMAX>(a, bv, bi, stream);
    case 12: return launch_bf16_rows<12, ARGMAX>(a, bv, bi, stream);
    case 13: return launch_bf16_rows<13, ARGMAX>(a, bv, bi, stream);
    case 14: return launch_bf16_rows<14, ARGMAX>(a, bv, bi, stream);
    case 15: return launch_bf16_rows<15, ARGMAX>(a, bv, bi, stream);
    case 16: return launch_bf16_rows<16, ARGMAX>(a, bv, bi, stream);
    default: return -1;
  }
}

constexpr int kMaxFastKBf16 = 512 * 16;
constexpr int kMaxFastKW8 = 1024 * 8;

bool bf16_fast_ok(const uint16_t* w, const uint16_t* x, int k) {
  return k >= 8 && (k & 7) == 0 && k <= kMaxFastKBf16 && aligned16(w) && aligned16(x);
}

bool w8_fast_ok(const int8_t* w, const uint16_t* x, int k) {
  return k >= 64 && (k & 63) == 0 && k <= kMaxFastKW8 && aligned16(w) && aligned16(x);
}

int generic_blocks(int tokens, int n) {
  const long long waves = static_cast<long long>(tokens) * n;
  const long long blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  return static_cast<int>(blocks < 65536 ? blocks : 65536);
}

}  // namespace

// ------------------------------------------------------ internal entries --

void launch_w8a16_gemv_fast(const W8GemvArgs& a, hipStream_t stream) {
  switch ((a.k + 1023) / 1024) {
    case 1: launch_w8_rows<1>(a, stream); break;
    case 2: launch_w8_rows<2>(a, stream); break;
    case 3: launch_w8_rows<3>(a, stream); break;
    case 4: launch_w8_rows<4>(a, stream); break;
    case 5: launch_w8_rows<5>(a, stream); break;
    case 6: launch_w8_rows<6>(a, stream); break;
    case 7: launch_w8_rows<7>(a, stream); break;
    case 8: launch_w8_rows<8>(a, stream); break;
    default: break;
  }
}

bool w8a16_gemv_fast_supported(const int8_t* w, const uint16_t* x, int k) {
  return w8_fast_ok(w, x, k);
}

int w8a16_slot_class(int k) { return (k + 1023) / 1024; }

// Rows per block of the grouped kernel for each slot class: 2 row steps per
// wave, RB = 4 / 2 / 1 rows per step for S = 1 / 2 / >= 3.
namespace {
constexpr int kGroupedSteps = 2;
constexpr int grouped_rb(int s) { return s == 1 ? 4 : (s == 2 ? 2 : 1); }

template <int S>
void launch_grouped(const W8GroupDesc* descs, int count, int blocks, hipStream_t stream) {
  hipLaunchKernelGGL((w8a16_gemv_grouped_kernel<S, grouped_rb(S), kGroupedSteps>), dim3(blocks),
                     dim3(kBlock), 0, stream, descs, count);
}
}  // namespace

int w8a16_grouped_rows_per_block(int slot_class) {
  return kWavesPerBlock * grouped_rb(slot_class) * kGroupedSteps;
}

void launch_w8a16_gemv_grouped(int slot_class, const W8GroupDesc* descs, int count,
                               int total_blocks, hipStream_t stream) {
  switch (slot_class) {
    case 1: launch_grouped<1>(descs, count, total_blocks, stream); break;
    case 2: launch_grouped<2>(descs, count, total_blocks, stream); break;
    case 3: launch_grouped<3>(descs, count, total_blocks, stream); break;
    case 4: launch_grouped<4>(descs, count, total_blocks, stream); break;
    case 5: launch_grouped<5>(descs, count, total_blocks, stream); break;
    case 6: launch_grouped<6>(descs, count, total_blocks, stream); break;
    case 7: launch_grouped<7>(descs, count, total_blocks, stream); break;
    case 8: launch_grouped<8>(descs, count, total_blocks, stream); break;
    default: break;
  }
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
  if (vocab <= 0 || in_features <= 0) return 0;
  const int cap = argmax_block_cap(vocab);
  int blocks;
  if (!fast) {
    blocks = generic_blocks(1, vocab);
  } else {
    const int s = (in_features + 511) / 512;
    const int rb = (s <= 4 && vocab >= 2048) ? 4 : ((s <= 8 && vocab >= 1024) ? 2 : 1);
    blocks = grid_for((vocab + rb - 1) / rb);
  }
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

extern "C" int infer_hip_lm_head_bf16(const uint16_t* weight, const uint16_t* bias,
                                      const uint16_t* input, uint16_t* logits,
                                      float* block_max_value, int* block_max_index, int* argmax,
                                      int vocab, int in_features, hipStream_t stream) {
  if (vocab <= 0 || in_features < 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "lm_head_bf16: bad shape V=%d K=%d", vocab,
                in_features);
  }
  if (!logits || !block_max_value || !block_max_index || !argmax ||
      (in_features > 0 && (!weight || !input))) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "lm_head_bf16: null required pointer");
  }
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
  hipLaunchKernelGGL(argmax_reduce_kernel, dim3(1), dim3(kBlock), 0, stream, block_max_value,
                     block_max_index, blocks, argmax);
  return check_launch("lm_head_bf16 argmax");
}
