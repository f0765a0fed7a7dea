// Device-side helpers shared by the Linear kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qlin {

constexpr int kWave = 64;

// BF16 word -> FP32: the word is the high half of the float.
__device__ __forceinline__ float bf16_to_f32(uint32_t word) {
  return __uint_as_float(word << 16);
}
// Low / high BF16 of a packed pair -> FP32 (one VALU op each).
__device__ __forceinline__ float bf16_lo(uint32_t pair) {
  return __uint_as_float(pair << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t pair) {
  return __uint_as_float(pair & 0xFFFF0000u);
}

// FP32 -> BF16 round-to-nearest-even; a NaN keeps its high half with the
// quiet bit set (the rounding the reference states at
// tools/export_model.py:123-131 and uses in its kernels).  gfx950's
// v_cvt_pk_bf16_f32 implements exactly this rounding — checked bit for bit
// against the add-0x7FFF-plus-lsb-and-truncate method over 2^26 random,
// tie, denormal, infinite and NaN inputs — without the per-value NaN
// branch of the integer method.
__device__ __forceinline__ uint16_t f32_to_bf16(float value) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(value));
}
// Two FP32 values -> a BF16 pair (lo in bits 0-15), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// e^x for x <= 0 (softmax weights) as the hardware's 2^(x log2(e)): two
// instructions where expf's range reduction takes ~12; within a few FP32
// ulps of expf (results below 2^-126 may flush to zero).
__device__ __forceinline__ float exp_nonpos_fast(float x) {
  return __builtin_amdgcn_exp2f(x * 1.44269504088896340736f);
}

// silu(g) * u = g / (1 + e^-g) * u on the hardware's 2^x and reciprocal
// (v_exp_f32 of -g log2(e), v_rcp_f32): six instructions where expf and the
// correctly rounded division take ~30.  Within a few FP32 ulps of the
// correctly rounded expression, so its BF16 rounding differs by one unit on
// about 1e-4 of the outputs; the GEMM epilogues that write many SiLU-mul
// outputs per thread use it.  g = -inf gives NaN as the division does; for
// g below about -87 the reciprocal of e^-g is subnormal and may be flushed,
// giving 0 where the division gives a value under 1e-36.
__device__ __forceinline__ float silu_mul_fast(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896340736f);
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// Pack two FP32 values, already exactly representable in BF16 (for example
// small integers), into a BF16 pair by truncation: lo in bits 0-15.
__device__ __forceinline__ uint32_t pack_bf16_trunc(float lo, float hi) {
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
}

// Sign-extended byte b of a dword, as FP32.  hipcc lowers each of these to a
// single v_cvt_f32_i32 with an SDWA byte select.
__device__ __forceinline__ float sbyte0(uint32_t v) {
  return static_cast<float>(static_cast<int8_t>(v));
}
__device__ __forceinline__ float sbyte1(uint32_t v) {
  return static_cast<float>(static_cast<int8_t>(v >> 8));
}
__device__ __forceinline__ float sbyte2(uint32_t v) {
  return static_cast<float>(static_cast<int8_t>(v >> 16));
}
__device__ __forceinline__ float sbyte3(uint32_t v) {
  return static_cast<float>(static_cast<int>(v) >> 24);
}

// Cross-lane moves without LDS.  dpp_from<CTRL> reads v from the lane the
// DPP control selects within the lane's row of 16 (quad permutes, row
// mirrors); rows_swapped16 / rows_swapped32 add the value of the lane 16 / 32
// rows away through gfx950's v_permlane16_swap / v_permlane32_swap: each swap
// exchanges half of one operand with half of the other, and with both
// operands = v the two results together hold the lane's row and its partner
// row, so their sum is the pair's total in every lane.  All lanes of the wave
// must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_from(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

constexpr int kDppQuadSwap1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

// Sum over the 64 lanes of a wave; every lane receives the total (the same
// total, summed in a fixed order).
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_from<kDppQuadSwap1>(v);
  v += dpp_from<kDppQuadSwap2>(v);
  v += dpp_from<kDppRowHalfMirror>(v);
  v += dpp_from<kDppRowMirror>(v);
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false,
                                                    false);
  v = __int_as_float(r16[0]) + __int_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false,
                                                    false);
  return __int_as_float(r32[0]) + __int_as_float(r32[1]);
}

// Maximum over the 64 lanes of a wave; every lane receives it.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_from<kDppQuadSwap1>(v));
  v = fmaxf(v, dpp_from<kDppQuadSwap2>(v));
  v = fmaxf(v, dpp_from<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp_from<kDppRowMirror>(v));
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false,
                                                    false);
  v = fmaxf(__int_as_float(r16[0]), __int_as_float(r16[1]));
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false,
                                                    false);
  return fmaxf(__int_as_float(r32[0]), __int_as_float(r32[1]));
}

// Sum within each row of 16 lanes; every lane of the row receives it.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_from<kDppQuadSwap1>(v);
  v += dpp_from<kDppQuadSwap2>(v);
  v += dpp_from<kDppRowHalfMirror>(v);
  return v + dpp_from<kDppRowMirror>(v);
}

// The lanes 32 (16) apart, exchanged between two values: with a and b the
// values of rows {0,1} and {2,3} (or of rows {0,2} and {1,3}), the sum
// returned is a's pair total in the lanes that keep a and b's in the others
// (gfx950 v_permlane32_swap / v_permlane16_swap).
__device__ __forceinline__ float swap32_sum(float a, float b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(a), __float_as_int(b), false,
                                                  false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}
__device__ __forceinline__ float swap16_sum(float a, float b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(a), __float_as_int(b), false,
                                                  false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}

// Reduce RB per-lane partials (one per row) across the wave with a
// reduce-scatter: each halving step hands half of the rows to the lanes 32,
// then 16, apart (permlane swaps for RB <= 4, shuffles beyond), and the
// remaining lanes of a group are summed (DPP within rows of 16).  On return
// vals[0] in every lane holds the total of row `reduced_row(lane)`.  All
// lanes must be active.
template <int RB>
__device__ __forceinline__ void wave_reduce_rows(float (&vals)[RB], int lane) {
  static_assert(RB >= 1 && RB <= 64 && (RB & (RB - 1)) == 0, "RB power of 2");
  if constexpr (RB == 1) {
    vals[0] = wave_sum(vals[0]);
    return;
  } else if constexpr (RB == 2) {
    // lanes 0-31 keep row 0, 32-63 row 1; then the 32 lanes of each half.
    const float h = swap32_sum(vals[0], vals[1]);
    vals[0] = row16_sum(swap16_sum(h, h));
    return;
  } else if constexpr (RB == 4) {
    // lanes 0-31 keep rows 0 and 1, 32-63 rows 2 and 3; then rows of 16
    // lanes: 0-15 / 32-47 keep the even row, 16-31 / 48-63 the odd one.
    const float a = swap32_sum(vals[0], vals[2]);
    const float b = swap32_sum(vals[1], vals[3]);
    vals[0] = row16_sum(swap16_sum(a, b));
    return;
  } else {
    int count = RB;
    int offset = 32;
#pragma unroll
    for (int step = RB; step > 1; step >>= 1) {
      const int half = count >> 1;
      const bool upper = (lane & offset) != 0;
#pragma unroll
      for (int i = 0; i < step / 2; ++i) {
        const float send = upper ? vals[i] : vals[i + half];
        const float keep = upper ? vals[i + half] : vals[i];
        vals[i] = keep + __shfl_xor(send, offset);
      }
      count = half;
      offset >>= 1;
    }
#pragma unroll
    for (; offset > 0; offset >>= 1) vals[0] += __shfl_xor(vals[0], offset);
  }
}

// Row index (0..RB-1) whose total wave_reduce_rows leaves in this lane.
template <int RB>
__device__ __forceinline__ int reduced_row(int lane) {
  int row = 0;
  int offset = 32;
#pragma unroll
  for (int step = RB; step > 1; step >>= 1) {
    if (lane & offset) row += step >> 1;
    offset >>= 1;
  }
  return row;
}

// The lane that writes row `reduced_row(lane)`: the lowest lane of each
// group of 64 / RB lanes.
template <int RB>
__device__ __forceinline__ bool is_row_writer(int lane) {
  return (lane & (kWave / RB - 1)) == 0;
}

// RoPE of one pair (a, b) = (x[i], x[i + head_dim / 2]) of a head by the
// angle whose (cos, sin) is cs (src/cpu_ops.cpp:33-56).
__device__ __forceinline__ void rope_pair(float& a, float& b, float2 cs) {
  const float first = a, second = b;
  a = first * cs.x - second * cs.y;
  b = second * cs.x + first * cs.y;
}

// Global-address-space access.  Pointers that reach a kernel through memory
// (a descriptor table) are generic to the compiler, which would then emit
// FLAT instructions; these casts keep every access a global_* instruction.
#define QLIN_GLOBAL __attribute__((address_space(1)))

template <typename T>
__device__ __forceinline__ T gload(const T* p) {
  return *(const QLIN_GLOBAL T*)(p);
}
template <typename T>
__device__ __forceinline__ void gstore(T* p, T v) {
  *(QLIN_GLOBAL T*)(p) = v;
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 16-byte global load.
__device__ __forceinline__ uint4 load_global16(const void* p) {
  const u32x4 v = *(const QLIN_GLOBAL u32x4*)(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// 16-byte global store.
__device__ __forceinline__ void store_global16(void* p, uint4 v) {
  *(QLIN_GLOBAL u32x4*)(p) = u32x4{v.x, v.y, v.z, v.w};
}

// 16-byte global load marked as streaming (the weights are read once per
// call, so they should not displace reused lines).
__device__ __forceinline__ uint4 load_stream16(const void* p) {
  const u32x4 v = __builtin_nontemporal_load((const QLIN_GLOBAL u32x4*)(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ------------------------------------------------- GEMV building blocks --

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
  const uint4 a = load_global16(x);
  const uint4 b = load_global16(x + 8);
  out[0] = bf16_lo(a.x);  out[1] = bf16_hi(a.x);
  out[2] = bf16_lo(a.y);  out[3] = bf16_hi(a.y);
  out[4] = bf16_lo(a.z);  out[5] = bf16_hi(a.z);
  out[6] = bf16_lo(a.w);  out[7] = bf16_hi(a.w);
  out[8] = bf16_lo(b.x);  out[9] = bf16_hi(b.x);
  out[10] = bf16_lo(b.y); out[11] = bf16_hi(b.y);
  out[12] = bf16_lo(b.z); out[13] = bf16_hi(b.z);
  out[14] = bf16_lo(b.w); out[15] = bf16_hi(b.w);
}

__device__ __forceinline__ void load_x8(const uint16_t* x, float (&out)[8]) {
  const uint4 a = load_global16(x);
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

// ------------------------------------------ device-coherent data exchange --
//
// Workgroups that hand data to each other inside one launch (split-K
// partials, attention partials, argmax candidates) store and load it with
// the sc1 cache policy: the accesses are coherent across the XCDs' separate
// L2 caches without the L2 write-back / invalidate a release / acquire
// fence would cost.  The hand-off itself is an agent-scope atomic counter
// taken after the stores have completed (s_waitcnt).
constexpr int kCoherentPolicy = 16;  // buffer cache policy bits: sc1

__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void* base,
                                                                 uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           0x00020000);
}

__device__ __forceinline__ void coherent_store(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset,
                                               float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, byte_offset, 0, kCoherentPolicy);
}

__device__ __forceinline__ void coherent_store(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset,
                                               int v) {
  __builtin_amdgcn_raw_buffer_store_b32(static_cast<uint32_t>(v), r, byte_offset, 0,
                                        kCoherentPolicy);
}

// Out-of-range offsets (beyond the resource's byte count) read 0.
__device__ __forceinline__ float coherent_load_f32(__amdgpu_buffer_rsrc_t r,
                                                   uint32_t byte_offset) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, byte_offset, 0, kCoherentPolicy));
}

__device__ __forceinline__ int coherent_load_i32(__amdgpu_buffer_rsrc_t r, uint32_t byte_offset) {
  return static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(r, byte_offset, 0, kCoherentPolicy));
}

}  // namespace qlin
