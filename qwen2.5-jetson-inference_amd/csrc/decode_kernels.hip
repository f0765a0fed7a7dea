// Fused decode-step kernels for gfx950: the GEMVs of a decode step (W8A16 or
// BF16 weights) with the RMSNorm in front of them (and the SiLU-mul behind
// gate/up) folded in, and the tied LM head with the final RMSNorm, the argmax
// and the step's bookkeeping folded in.
//
// A decode step is latency-bound: every kernel starts on a cold L2 and each
// dependent global round trip costs about a microsecond, so these kernels
// are built to need one round trip: a wave issues its weight loads, then its
// activation and norm-weight loads (all independent), and only then waits.
// With K <= 64 C x SLABS, the 64 lanes of one wave hold the whole input
// vector (lane l owns C-element chunks l, l + 64, ..., where C = 16 for
// int8 weights and 8 for BF16: one 16-byte weight load each), so each wave
// computes the RMSNorm of x by itself: no workgroup reduction, no extra
// launch, no normalized copy in memory.
//
// Numerics follow the unfused ops exactly in kind (not in summation order):
// the normalized activations are rounded to BF16 as rms_norm_bf16 stores
// them (src/cuda/kernels.cu:64-116), gate and up are rounded to BF16 before
// silu_mul (kernels.cu:302-324), the LM head argmax is over the FP32 sums
// with ties to the lowest index (kernels.cu:492-603).
#include <float.h>
#include <limits.h>
#include <stdint.h>

#include "decode_kernels.hpp"
#include "model_kernels.hpp"
#include "device_common.hpp"

namespace qlin {

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;

// Branch-free loads.  Every load of these kernels is issued unconditionally
// from a clamped index (a row past the matrix reads its last row, a chunk
// past K its last chunk) and the value is masked afterwards, so that no
// branch separates the loads: the compiler would otherwise wait for each
// branch's loads before leaving it and serialise the weight and activation
// round trips.  Kernels issue their weight loads first, then the activation
// loads, then a scheduling barrier, then compute.

// Raw 16-byte chunks of a BF16 vector of k values: 8 values per chunk,
// lane l holding chunk s * 64 + l of slab s (clamped).
template <int SLABS>
__device__ __forceinline__ void load_vec8_raw(const uint16_t* v, int k, int lane,
                                              uint4 (&raw)[SLABS]) {
  const int chunks = k >> 3;
#pragma unroll
  for (int s = 0; s < SLABS; ++s) {
    raw[s] = load_global16(v + 8 * min(s * kWave + lane, chunks - 1));
  }
}

// 16-value chunks: two 16-byte halves per chunk.
template <int SLABS>
__device__ __forceinline__ void load_vec16_raw(const uint16_t* v, int k, int lane,
                                               uint4 (&lo)[SLABS], uint4 (&hi)[SLABS]) {
  const int chunks = k >> 4;
#pragma unroll
  for (int s = 0; s < SLABS; ++s) {
    const int c = min(s * kWave + lane, chunks - 1);
    lo[s] = load_global16(v + 16 * c);
    hi[s] = load_global16(v + 16 * c + 8);
  }
}

// Raw chunks of C values (C = 8 or 16: C / 8 16-byte pieces per chunk).
template <int C, int SLABS>
__device__ __forceinline__ void load_vec_raw(const uint16_t* v, int k, int lane,
                                             uint4 (&raw)[SLABS][C / 8]) {
  if constexpr (C == 16) {
    uint4 lo[SLABS], hi[SLABS];
    load_vec16_raw<SLABS>(v, k, lane, lo, hi);
#pragma unroll
    for (int s = 0; s < SLABS; ++s) {
      raw[s][0] = lo[s];
      raw[s][1] = hi[s];
    }
  } else {
    uint4 r[SLABS];
    load_vec8_raw<SLABS>(v, k, lane, r);
#pragma unroll
    for (int s = 0; s < SLABS; ++s) raw[s][0] = r[s];
  }
}

__device__ __forceinline__ void unpack8(const uint4 w, bool keep, float* out) {
  out[0] = keep ? bf16_lo(w.x) : 0.0f; out[1] = keep ? bf16_hi(w.x) : 0.0f;
  out[2] = keep ? bf16_lo(w.y) : 0.0f; out[3] = keep ? bf16_hi(w.y) : 0.0f;
  out[4] = keep ? bf16_lo(w.z) : 0.0f; out[5] = keep ? bf16_hi(w.z) : 0.0f;
  out[6] = keep ? bf16_lo(w.w) : 0.0f; out[7] = keep ? bf16_hi(w.w) : 0.0f;
}

// The wave's RMSNorm of x (chunks of C values, C = 8 or 16, already loaded
// raw) rounded to BF16, zero past K.
template <int SLABS, int C>
__device__ __forceinline__ void wave_rms_norm(const uint4 (&xr)[SLABS][C / 8],
                                              const uint4 (&nr)[SLABS][C / 8], int k, float eps,
                                              int lane, float (&xn)[SLABS][C]) {
  const int chunks = k / C;
  float nw[SLABS][C];
#pragma unroll
  for (int s = 0; s < SLABS; ++s) {
    const bool keep = s * kWave + lane < chunks;
#pragma unroll
    for (int h = 0; h < C / 8; ++h) {
      unpack8(xr[s][h], keep, &xn[s][8 * h]);
      unpack8(nr[s][h], true, &nw[s][8 * h]);
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int s = 0; s < SLABS; ++s)
#pragma unroll
    for (int e = 0; e < C; ++e) ss = fmaf(xn[s][e], xn[s][e], ss);
  ss = wave_sum(ss);
  const float scale = 1.0f / sqrtf(ss / k + eps);
#pragma unroll
  for (int s = 0; s < SLABS; ++s)
#pragma unroll
    for (int e = 0; e < C; ++e) xn[s][e] = bf16_to_f32(f32_to_bf16(xn[s][e] * scale * nw[s][e]));
}

// Raw int8 chunks and group scales of one row (clamped row and chunks).
template <int SLABS>
__device__ __forceinline__ void load_w8_row(const int8_t* w, const uint16_t* s, int row, int n,
                                            int k, int lane, uint4 (&wq)[SLABS],
                                            uint32_t (&sc)[SLABS]) {
  const int chunks = k >> 4, groups = k >> 6;
  const int r = min(row, n - 1);
#pragma unroll
  for (int i = 0; i < SLABS; ++i) {
    const int c = min(i * kWave + lane, chunks - 1);
    wq[i] = load_stream16(w + static_cast<size_t>(r) * k + 16 * c);
    sc[i] = gload(s + static_cast<size_t>(r) * groups + (c >> 2));
  }
}

// The row's dot product with the activations, summed over the wave.  The
// scales of chunks past K (or of a row past the matrix) are taken as 0;
// the int8 weights are finite, so those chunks add exactly 0.
template <int SLABS>
__device__ __forceinline__ float w8_row_dot(const uint4 (&wq)[SLABS], const uint32_t (&sc)[SLABS],
                                            const float (&xn)[SLABS][16], bool row_ok, int k,
                                            int lane) {
  const int chunks = k >> 4;
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < SLABS; ++i) {
    const float scale = row_ok && i * kWave + lane < chunks ? bf16_to_f32(sc[i]) : 0.0f;
    acc = fmaf(dot16_i8(wq[i], xn[i]), scale, acc);
  }
  return wave_sum(acc);
}

// Weight formats of the fused GEMVs.  A row is read as 16-byte chunks, lane
// l holding chunks l, l + 64, ... (SLABS of them), all requested at once.
//
// W8A16: 16 int8 weights per chunk and the BF16 scale of its 64-group;
// chunk sums are scaled per chunk (dot16_i8, then the scale), as the
// unfused W8A16 GEMV does.
struct W8Fmt {
  static constexpr int C = 16;
  template <int SLABS>
  struct Row {
    uint4 q[SLABS];
    uint32_t s[SLABS];
  };
  template <int SLABS>
  static __device__ __forceinline__ void load(const void* w, const uint16_t* s, int row, int n,
                                              int k, int lane, Row<SLABS>& r) {
    load_w8_row<SLABS>(static_cast<const int8_t*>(w), s, row, n, k, lane, r.q, r.s);
  }
  template <int SLABS>
  static __device__ __forceinline__ float dot(const Row<SLABS>& r, const float (&x)[SLABS][C],
                                              bool row_ok, int k, int lane) {
    return w8_row_dot<SLABS>(r.q, r.s, x, row_ok, k, lane);
  }
};

// BF16: 8 weights per chunk, no scales.  Chunks past K (or a row past the
// matrix) re-read the last chunk (row) and are discarded by a select, so
// whatever they hold cannot reach the sum.
struct Bf16Fmt {
  static constexpr int C = 8;
  template <int SLABS>
  struct Row {
    uint4 q[SLABS];
  };
  template <int SLABS>
  static __device__ __forceinline__ void load(const void* w, const uint16_t*, int row, int n,
                                              int k, int lane, Row<SLABS>& r) {
    const uint16_t* wb = static_cast<const uint16_t*>(w);
    const int chunks = k >> 3;
    const int rr = min(row, n - 1);
#pragma unroll
    for (int i = 0; i < SLABS; ++i) {
      const int c = min(i * kWave + lane, chunks - 1);
      r.q[i] = load_stream16(wb + static_cast<size_t>(rr) * k + 8 * c);
    }
  }
  template <int SLABS>
  static __device__ __forceinline__ float dot(const Row<SLABS>& r, const float (&x)[SLABS][C],
                                              bool row_ok, int k, int lane) {
    const int chunks = k >> 3;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < SLABS; ++i) {
      const float next = dot8_bf16(r.q[i], x[i], acc);
      acc = row_ok && i * kWave + lane < chunks ? next : acc;
    }
    return wave_sum(acc);
  }
};

// Descriptor of the workgroup: the last one whose block_begin <= b.
__device__ __forceinline__ NormGemvDesc pick_desc(const NormGemvArgs& a, int b) {
  NormGemvDesc d = a.d[0];
  if (a.count > 1 && a.d[1].block_begin <= b) d = a.d[1];
  if (a.count > 2 && a.d[2].block_begin <= b) d = a.d[2];
  return d;
}

}  // namespace

// y = bf16(W(rms_norm(x)) + bias) for up to three GEMVs on the same
// normalized input (q|k|v), or with PAIR mlp = bf16(silu(bf16(gate)) *
// bf16(up)) from the gate (w, s) and up (w2, s2) rows of the same index.
// Each wave computes R consecutive output rows (all their loads in flight
// together); 4 R rows per workgroup.  F is the weight format (W8Fmt,
// Bf16Fmt).
template <class F, int SLABS, bool PAIR, int R>
__global__ __launch_bounds__(kBlock) void norm_gemv_kernel(NormGemvArgs a) {
  constexpr int C = F::C;
  const NormGemvDesc d = pick_desc(a, blockIdx.x);
  const int lane = threadIdx.x & (kWave - 1);
  const int row0 = ((blockIdx.x - d.block_begin) * kWaves + threadIdx.x / kWave) * R;
  // x and the RMSNorm weight first: loads return in the order they were
  // issued, so the normalization then runs while the weights stream in
  // (measured: gate|up 4.95 -> 4.53 us per launch)
  uint4 xr[SLABS][C / 8], nr[SLABS][C / 8];
  load_vec_raw<C, SLABS>(a.x, a.k, lane, xr);
  load_vec_raw<C, SLABS>(a.norm_w, a.k, lane, nr);
  typename F::template Row<SLABS> w1[R], w2[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    F::template load<SLABS>(d.w, d.s, row0 + r, d.n, a.k, lane, w1[r]);
    if (PAIR) F::template load<SLABS>(d.w2, d.s2, row0 + r, d.n, a.k, lane, w2[r]);
  }
  // The bias of the row this lane writes (lane r < R), requested with the
  // weights so the store at the end waits on no further round trip; an
  // absent bias reads y instead and is discarded.
  const int brow = min(row0 + min(lane, R - 1), d.n - 1);
  const uint16_t bias_raw = gload((d.bias && !PAIR ? d.bias : d.y) + brow);
  __builtin_amdgcn_sched_barrier(0);  // every load is in flight
  float xn[SLABS][C];
  wave_rms_norm<SLABS, C>(xr, nr, a.k, a.eps, lane, xn);
  float v1[R], v2[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bool ok = row0 + r < d.n;
    v1[r] = F::template dot<SLABS>(w1[r], xn, ok, a.k, lane);
    if (PAIR) v2[r] = F::template dot<SLABS>(w2[r], xn, ok, a.k, lane);
  }
  if (lane < R) {
    // Lane r writes row row0 + r (every lane holds every total).
    float g = v1[0], u = PAIR ? v2[0] : 0.0f;
#pragma unroll
    for (int r = 1; r < R; ++r) {
      if (lane == r) {
        g = v1[r];
        if (PAIR) u = v2[r];
      }
    }
    const int row = row0 + lane;
    if (row < d.n) {
      if (PAIR) {
        const float gb = bf16_to_f32(f32_to_bf16(g));
        const float ub = bf16_to_f32(f32_to_bf16(u));
        gstore(d.y + row, f32_to_bf16(gb / (1.0f + expf(-gb)) * ub));
      } else {
        const float b = d.bias ? bf16_to_f32(bias_raw) : 0.0f;
        gstore(d.y + row, f32_to_bf16(g + b));
      }
    }
  }
}

// q|k|v with the RMSNorm in front and the RoPE and KV-cache store behind
// (QkvRopeArgs).  One wave per pair of output rows, all loads issued
// before the first wait: (i, i + head_dim / 2) of a q or k head (the pair
// the rotation mixes, so a lane holds both sums), or two consecutive rows
// of v.  Tasks are the q pairs, then the k pairs, then the v pairs.  The
// position is read at entry and its (cos, sin) requested once it arrives,
// behind the weight loads, so the rotation waits on no extra round trip.
// F is the weight format (W8Fmt, Bf16Fmt).
template <class F, int SLABS>
__global__ __launch_bounds__(kBlock) void norm_qkv_rope_kernel(QkvRopeArgs a) {
  constexpr int C = F::C;
  const int lane = threadIdx.x & (kWave - 1);
  const int half = a.head_dim / 2;
  const int qt = a.heads * half, kt = a.kv_heads * half;
  const int total = qt + 2 * kt;
  // wave-uniform (scalar registers for the task's pointers and rows)
  const int task = __builtin_amdgcn_readfirstlane(
      min(static_cast<int>(blockIdx.x) * kWaves + static_cast<int>(threadIdx.x) / kWave,
          total - 1));
  const int region = task < qt ? 0 : task < qt + kt ? 1 : 2;  // q, k, v
  const int t = task - (region == 0 ? 0 : region == 1 ? qt : qt + kt);
  const void* w = region == 0 ? a.wq : region == 1 ? a.wk : a.wv;
  const uint16_t* sc = region == 0 ? a.sq : region == 1 ? a.sk : a.sv;
  const uint16_t* bias = region == 0 ? a.bq : region == 1 ? a.bk : a.bv;
  const int n = region == 0 ? a.heads * a.head_dim : a.kv_heads * a.head_dim;
  // rows of the pair: (head * hd + i, + half) for q and k, (2 t, 2 t + 1) for v
  const int head = t / half, i = t % half;
  const int r0 = region == 2 ? 2 * t : head * a.head_dim + i;
  const int r1 = region == 2 ? 2 * t + 1 : r0 + half;
  // A negative position is an empty context: k and v are not stored
  // (the attention kernels read nothing for it either).
  const int raw_pos = *a.pos;
  const int pos = min(raw_pos, a.max_seq - 1);
  // x and the RMSNorm weight first, so the normalization runs while the
  // weights stream in (loads return in issue order)
  uint4 xr[SLABS][C / 8], nr[SLABS][C / 8];
  load_vec_raw<C, SLABS>(a.x, a.k, lane, xr);
  load_vec_raw<C, SLABS>(a.norm_w, a.k, lane, nr);
  typename F::template Row<SLABS> w0, w1;
  F::template load<SLABS>(w, sc, r0, n, a.k, lane, w0);
  F::template load<SLABS>(w, sc, r1, n, a.k, lane, w1);
  // the biases of r0 and r1 (an absent bias reads weight bytes instead, discarded)
  const uint16_t* bsrc = bias ? bias : static_cast<const uint16_t*>(w);
  const uint16_t bias_raw0 = gload(bsrc + r0), bias_raw1 = gload(bsrc + r1);
  const float2 cs = a.rope_row[i];
  __builtin_amdgcn_sched_barrier(0);  // every load is in flight
  float xn[SLABS][C];
  wave_rms_norm<SLABS, C>(xr, nr, a.k, a.eps, lane, xn);
  const float v0 = F::template dot<SLABS>(w0, xn, true, a.k, lane);
  const float v1 = F::template dot<SLABS>(w1, xn, true, a.k, lane);
  const float b = bias ? bf16_to_f32(bias_raw0) : 0.0f;
  const float b1 = bias ? bf16_to_f32(bias_raw1) : 0.0f;
  if (lane == 0 && static_cast<int>(blockIdx.x) * kWaves + static_cast<int>(threadIdx.x) / kWave <
                       total) {
    float y0 = bf16_to_f32(f32_to_bf16(v0 + b));
    float y1 = bf16_to_f32(f32_to_bf16(v1 + b1));
    if (region != 2) rope_pair(y0, y1, cs);
    const uint16_t o0 = f32_to_bf16(y0), o1 = f32_to_bf16(y1);
    if (region == 0) {
      gstore(a.q_out + r0, o0);
      gstore(a.q_out + r1, o1);
    } else if (raw_pos >= 0) {
      // row r of k or v is dimension r % head_dim of kv head r / head_dim
      uint16_t* cache = region == 1 ? a.key_cache : a.value_cache;
      const size_t base = (static_cast<size_t>(r0 / a.head_dim) * a.max_seq + pos) * a.head_dim;
      gstore(cache + base + r0 % a.head_dim, o0);
      gstore(cache + base + r1 % a.head_dim, o1);
    }
  }
}

// One GEMV row per wave, all K chunks of the row requested at once (lane
// l: chunks l, l + 64, ...), with the residual add: y[row] = bf16(W[row] .
// x + bias[row]); bias may alias y (each element is read and then written
// by the same lane).  F is the weight format (W8Fmt, Bf16Fmt).
template <class F, int SLABS>
__global__ __launch_bounds__(kBlock) void gemv_rows_kernel(GemvRowsArgs a) {
  constexpr int C = F::C;
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * kWaves + threadIdx.x / kWave;
  // x first, so its conversion runs while the weights stream in (loads
  // return in issue order)
  uint4 xr[SLABS][C / 8];
  load_vec_raw<C, SLABS>(a.x, a.k, lane, xr);
  typename F::template Row<SLABS> wr;
  F::template load<SLABS>(a.w, a.s, row, a.n, a.k, lane, wr);
  // the bias (the residual, which this lane alone overwrites at the end)
  // with the other loads; an absent bias reads y instead and is discarded
  const uint16_t bias_raw = gload((a.bias ? a.bias : a.y) + min(row, a.n - 1));
  __builtin_amdgcn_sched_barrier(0);  // every load is in flight
  const int chunks = a.k >> (C == 16 ? 4 : 3);
  float xv[SLABS][C];
#pragma unroll
  for (int s = 0; s < SLABS; ++s) {
    const bool keep = s * kWave + lane < chunks;
#pragma unroll
    for (int h = 0; h < C / 8; ++h) unpack8(xr[s][h], keep, &xv[s][8 * h]);
  }
  const float v = F::template dot<SLABS>(wr, xv, row < a.n, a.k, lane);
  if (lane == 0 && row < a.n) {
    const float b = a.bias ? bf16_to_f32(bias_raw) : 0.0f;
    gstore(a.y + row, f32_to_bf16(v + b));
  }
}

// Slabs of 64 16-byte weight chunks spanning K (1024 int8 or 512 BF16
// weights each).
static int fused_slabs(int k, bool w8) {
  const int per_slab = kWave * (w8 ? W8Fmt::C : Bf16Fmt::C);
  return (k + per_slab - 1) / per_slab;
}

bool attn_o_parts_supported(int k, bool w8) {
  return k >= 64 && k % 64 == 0 && fused_slabs(k, w8) <= 4;
}

// The o-projection with the merge of the attention's P parts (two halves or
// four quarters; see decode_kernels.hpp).  The merge is done once per
// workgroup: its 256 threads each merge four consecutive attention outputs
// (rounds of 1024) from the P records, with the records' loads, the
// weight row's and the residual's in flight at once, and store them as BF16
// in LDS; after one barrier every wave reads its lanes' inputs from there
// (lane l's chunk c, C = 16 inputs for int8 weights, 8 for BF16).  A part
// that the context has not reached is never summed (select, so stale
// values cannot reach the result).  Measured at config 4 (quarters): 2.92
// us per launch against 3.37 when each wave merged every head from the
// records itself (four times the record loads, no barrier).  F is the
// weight format (W8Fmt, Bf16Fmt).
template <class F, int SLABS, int P>
__global__ __launch_bounds__(kBlock) void attn_o_parts_kernel(AttnOPartsArgs a) {
  constexpr int C = F::C;
  constexpr int S = kAttnWholeMax / P;  // positions per part
  constexpr int RQ = (SLABS * kWave * C / 4 + kBlock - 1) / kBlock;  // merge rounds
  __shared__ __align__(16) uint16_t xs[SLABS * kWave * C];
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int row = blockIdx.x * kWaves + tid / kWave;
  const int chunks = a.k / C, quads = a.k >> 2;
  const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(a.partial), 0, a.heads * P * kAttnPartRecord * 4, 0x00020000);
  float4 r[RQ][P];
  float2 ml[RQ][P];
#pragma unroll
  for (int q = 0; q < RQ; ++q) {
    const uint32_t i = static_cast<uint32_t>(min(q * kBlock + tid, quads - 1));
    const uint32_t b0 = (i / 16u) * P * kAttnPartRecord * 4u, d = (i % 16u) * 16u;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const uint32_t bp = b0 + p * kAttnPartRecord * 4u;
      r[q][p] = __builtin_bit_cast(float4,
                                   __builtin_amdgcn_raw_buffer_load_b128(pr, bp + d, 0, 0));
      ml[q][p] = __builtin_bit_cast(
          float2, __builtin_amdgcn_raw_buffer_load_b64(pr, bp + 64u * 4u, 0, 0));
    }
  }
  typename F::template Row<SLABS> wr;
  F::template load<SLABS>(a.w, a.s, row, a.n, a.k, lane, wr);
  const uint16_t res_raw = gload(a.x + min(row, a.n - 1));
  const int pos = min(*a.pos, a.max_seq - 1);
  __builtin_amdgcn_sched_barrier(0);  // every load is in flight
  const int live = pos / S + 1;       // parts [0, live) hold records
#pragma unroll
  for (int q = 0; q < RQ; ++q) {
    const int i = q * kBlock + tid;
    float m = ml[q][0].x;
#pragma unroll
    for (int p = 1; p < P; ++p) m = p < live ? fmaxf(m, ml[q][p].x) : m;
    float w[P];
#pragma unroll
    for (int p = 0; p < P; ++p) w[p] = p == 0 || p < live ? exp_nonpos_fast(ml[q][p].x - m) : 0.0f;
    float ll = ml[q][0].y * w[0];
#pragma unroll
    for (int p = 1; p < P; ++p) ll = p < live ? fmaf(ml[q][p].y, w[p], ll) : ll;
    const float inv = 1.0f / ll;
    float av[P][4];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      av[p][0] = r[q][p].x;
      av[p][1] = r[q][p].y;
      av[p][2] = r[q][p].z;
      av[p][3] = r[q][p].w;
    }
    float o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float aa = av[0][t] * w[0];
#pragma unroll
      for (int p = 1; p < P; ++p) aa = p < live ? fmaf(av[p][t], w[p], aa) : aa;
      o[t] = aa * inv;
    }
    if (i < quads) {
      // the attention's output is BF16, as attention_decode_bf16 stores it
      const uint2 packed = {f32_to_bf16(o[0]) | (static_cast<uint32_t>(f32_to_bf16(o[1])) << 16),
                            f32_to_bf16(o[2]) | (static_cast<uint32_t>(f32_to_bf16(o[3])) << 16)};
      *reinterpret_cast<uint2*>(xs + 4 * i) = packed;
    }
  }
  __syncthreads();
  float xv[SLABS][C];
#pragma unroll
  for (int s = 0; s < SLABS; ++s) {
    const int c = s * kWave + lane;
    const bool keep = c < chunks;
    const uint16_t* src = xs + C * min(c, chunks - 1);
#pragma unroll
    for (int j = 0; j < C / 8; ++j) {
      const uint4 u = *reinterpret_cast<const uint4*>(src + 8 * j);
      const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        xv[s][8 * j + 2 * t] = keep ? bf16_to_f32(wd[t] & 0xFFFFu) : 0.0f;
        xv[s][8 * j + 2 * t + 1] = keep ? bf16_to_f32(wd[t] >> 16) : 0.0f;
      }
    }
  }
  const float v = F::template dot<SLABS>(wr, xv, row < a.n, a.k, lane);
  if (lane == 0 && row < a.n) gstore(a.x + row, f32_to_bf16(v + bf16_to_f32(res_raw)));
}

template <class F, int P>
static void launch_attn_o_parts_fmt(const AttnOPartsArgs& a, hipStream_t stream) {
  const dim3 grid((a.n + kWaves - 1) / kWaves), block(kBlock);
  const int slabs = fused_slabs(a.k, F::C == W8Fmt::C);
  if (slabs <= 1) {
    hipLaunchKernelGGL((attn_o_parts_kernel<F, 1, P>), grid, block, 0, stream, a);
  } else if (slabs <= 2) {
    hipLaunchKernelGGL((attn_o_parts_kernel<F, 2, P>), grid, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL((attn_o_parts_kernel<F, 4, P>), grid, block, 0, stream, a);
  }
}

void launch_attn_o_parts(const AttnOPartsArgs& a, bool w8, hipStream_t stream, int parts) {
  if (parts == 4) {
    if (w8) {
      launch_attn_o_parts_fmt<W8Fmt, 4>(a, stream);
    } else {
      launch_attn_o_parts_fmt<Bf16Fmt, 4>(a, stream);
    }
  } else if (w8) {
    launch_attn_o_parts_fmt<W8Fmt, 2>(a, stream);
  } else {
    launch_attn_o_parts_fmt<Bf16Fmt, 2>(a, stream);
  }
}

// The tied LM head of a decode step: logits = bf16(E rms_norm(x)) with the
// argmax of the FP32 sums.  A grid of at most lm_head_decode_blocks()
// workgroups; each wave normalizes x once and walks R-row tasks with a
// stride of the grid's wave count, keeping the next task's loads in flight.
// R rows per task (1, 2, 4 or 8).
// Every workgroup leaves its best (value, index) pair; the last to finish
// (counted on `counter`) reduces them, writes the token to *token and, with
// `advance`, records it in history[state->step] and moves the step and
// position on by one.  It then resets the counter.
template <int SLABS, int R>
__global__ __launch_bounds__(kBlock) void lm_head_decode_kernel(LmHeadDecodeArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int chunks = a.k >> 3;
  float xn[SLABS][8];
  const int gw = blockIdx.x * kWaves + wave;
  const int stride = gridDim.x * kWaves * R;
  int row0 = gw * R;
  uint4 w[R][SLABS], wn[R][SLABS];
  auto load_task = [&](int r0, uint4 (&dst)[R][SLABS]) {
    // Clamped rows and chunks: past-the-end rows are not written, and past
    // K the activations are 0.
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(r0 + r, a.vocab - 1);
#pragma unroll
      for (int s = 0; s < SLABS; ++s) {
        const int c = min(s * kWave + lane, chunks - 1);
        dst[r][s] = load_stream16(a.w + static_cast<size_t>(row) * a.k + 8 * c);
      }
    }
  };
  {
    // x and the RMSNorm weight before the first task's rows: loads return
    // in issue order, so the normalization runs while the rows stream in
    uint4 xr[SLABS][1], nr[SLABS][1], raw[SLABS], add[SLABS];
    load_vec8_raw<SLABS>(a.x, a.k, lane, raw);
#pragma unroll
    for (int s = 0; s < SLABS; ++s) xr[s][0] = raw[s];
    // the residual to add first (x_add); without one, x again (unused): no
    // branch around a load
    load_vec8_raw<SLABS>(a.x_add ? a.x_add : a.x, a.k, lane, add);
    load_vec8_raw<SLABS>(a.norm_w, a.k, lane, raw);
#pragma unroll
    for (int s = 0; s < SLABS; ++s) nr[s][0] = raw[s];
    load_task(row0, w);
    __builtin_amdgcn_sched_barrier(0);  // every load is in flight
    if (a.x_add) {
#pragma unroll
      for (int s = 0; s < SLABS; ++s) {  // bf16(x + x_add), as add_kernel
        const uint4 x = xr[s][0], y = add[s];
        xr[s][0] = make_uint4(pack2_bf16(bf16_lo(x.x) + bf16_lo(y.x), bf16_hi(x.x) + bf16_hi(y.x)),
                              pack2_bf16(bf16_lo(x.y) + bf16_lo(y.y), bf16_hi(x.y) + bf16_hi(y.y)),
                              pack2_bf16(bf16_lo(x.z) + bf16_lo(y.z), bf16_hi(x.z) + bf16_hi(y.z)),
                              pack2_bf16(bf16_lo(x.w) + bf16_lo(y.w), bf16_hi(x.w) + bf16_hi(y.w)));
      }
    }
    wave_rms_norm<SLABS, 8>(xr, nr, a.k, a.eps, lane, xn);
  }
  // The (cos, sin) row of the next position, for the last workgroup when it
  // advances the state (requested by every workgroup, long before needed).
  const bool keep_rope =
      a.advance == 1 && a.rope.row && static_cast<int>(threadIdx.x) < a.rope.half;
  float2 rope_next = make_float2(0.0f, 0.0f);
  if (keep_rope) {
    rope_next = a.rope.table[static_cast<size_t>(min(a.state->pos + 1, a.rope.max_seq - 1)) *
                                 a.rope.half + threadIdx.x];
  }
  float best_v = -FLT_MAX;
  int best_i = INT_MAX;
  for (; row0 < a.vocab; row0 += stride) {
    load_task(row0 + stride, wn);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      acc[r] = 0.0f;
#pragma unroll
      for (int s = 0; s < SLABS; ++s) acc[r] = dot8_bf16(w[r][s], xn[s], acc[r]);
    }
    wave_reduce_rows<R>(acc, lane);
    if (is_row_writer<R>(lane)) {
      const int row = row0 + reduced_row<R>(lane);
      if (row < a.vocab) {
        gstore(a.logits + row, f32_to_bf16(acc[0]));
        if (better(acc[0], row, best_v, best_i)) {
          best_v = acc[0];
          best_i = row;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int s = 0; s < SLABS; ++s) w[r][s] = wn[r][s];
  }
  wave_argmax(best_v, best_i);
  __shared__ float wv[kWaves];
  __shared__ int wi[kWaves];
  __shared__ int last;
  if (lane == 0) {
    wv[wave] = best_v;
    wi[wave] = best_i;
  }
  __syncthreads();
  if (a.advance == 2) {
    if (threadIdx.x == 0) {
      float v = wv[0];
      int i = wi[0];
      for (int k = 1; k < kWaves; ++k) {
        if (better(wv[k], wi[k], v, i)) {
          v = wv[k];
          i = wi[k];
        }
      }
      // a workgroup whose rows never win the comparison (all NaN or -inf)
      // offers its first row at the lowest key, so such a vocabulary yields
      // row 0
      const unsigned long long k =
          i == INT_MAX ? lm_pack_key(__builtin_nanf(""), blockIdx.x * kWaves * R)
                       : lm_pack_key(v, i);
      __hip_atomic_fetch_max(a.key, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  const __amdgpu_buffer_rsrc_t cand =
      coherent_rsrc(a.block_best, static_cast<uint32_t>(gridDim.x) * 8u);
  if (threadIdx.x == 0) {
    float v = wv[0];
    int i = wi[0];
    for (int k = 1; k < kWaves; ++k) {
      if (better(wv[k], wi[k], v, i)) {
        v = wv[k];
        i = wi[k];
      }
    }
    coherent_store(cand, blockIdx.x * 8u, v);
    coherent_store(cand, blockIdx.x * 8u + 4u, i);
    __builtin_amdgcn_s_waitcnt(0);
    last = __hip_atomic_fetch_add(a.counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           static_cast<int>(gridDim.x) - 1;
  }
  __syncthreads();
  if (!last) return;
  // The last workgroup: reduce every workgroup's candidate.
  float v = -FLT_MAX;
  int i = INT_MAX;
  for (int b = threadIdx.x; b < static_cast<int>(gridDim.x); b += kBlock) {
    const float cv = coherent_load_f32(cand, b * 8u);
    const int ci = coherent_load_i32(cand, b * 8u + 4u);
    if (better(cv, ci, v, i)) {
      v = cv;
      i = ci;
    }
  }
  wave_argmax(v, i);
  if (lane == 0) {
    wv[wave] = v;
    wi[wave] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < kWaves; ++k) {
      if (better(wv[k], wi[k], wv[0], wi[0])) {
        wv[0] = wv[k];
        wi[0] = wi[k];
      }
    }
    *a.token = wi[0];
    if (a.advance) {
      ModelState* st = a.state;
      const int step = st->step;
      if (step < a.history_len) a.history[step] = wi[0];
      st->step = step + 1;
      st->pos = st->pos + 1;
    }
    __hip_atomic_store(a.counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (keep_rope) a.rope.row[threadIdx.x] = rope_next;
}


// The o-projection of a decode step fused with the merge of the split
// attention's partials and the residual add:
//   attn = bf16(merge of the ceil((pos + 1) / span) spans' partials)
//   x[row] = bf16(Wo[row] . attn + x[row])
// All 256 threads first request their weight row (one row per wave, four
// per workgroup) and the partials, then merge into LDS; the GEMV reads attn
// from LDS.  Records past a head's last split (stale, or other heads'
// records, or zeros past the buffer) are loaded with the rest but never
// enter a sum, so whatever they hold cannot reach the result.
template <int SLABS, bool W8, int MAXS, int R>
__global__ __launch_bounds__(kBlock) void attn_o_gemv_kernel(AttnOArgs a) {
  constexpr int kChunk = W8 ? 16 : 8;          // values per 16-byte weight chunk
  constexpr int kMaxK = SLABS * kWave * kChunk;
  constexpr int kPer = (kMaxK + kBlock - 1) / kBlock;
  __shared__ float attn[kMaxK];
  __shared__ float ms[kAttnOMaxHeads][MAXS], ls[kAttnOMaxHeads][MAXS];
  __shared__ float hw[kAttnOMaxHeads][MAXS];
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int row0 = (blockIdx.x * kWaves + tid / kWave) * R;
  const int chunks = a.k / kChunk;
  // Weight rows (R per wave).
  uint4 wq[R][SLABS];
  uint32_t sc[R][SLABS];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (W8) {
      load_w8_row<SLABS>(static_cast<const int8_t*>(a.w), a.s, row0 + r, a.n, a.k, lane, wq[r],
                         sc[r]);
    } else {
      const int rr = min(row0 + r, a.n - 1);
#pragma unroll
      for (int i = 0; i < SLABS; ++i) {
        const int c = min(i * kWave + lane, chunks - 1);
        wq[r][i] = load_stream16(static_cast<const uint16_t*>(a.w) +
                                 static_cast<size_t>(rr) * a.k + 8 * c);
      }
    }
  }
  // Partials.
  const int hd = a.head_dim, rec = hd + 2;
  const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(a.partial), 0, a.heads * a.max_splits * rec * 4, 0x00020000);
  float acc_s[kPer][MAXS];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int o = tid + kBlock * i;
    const int h = o / hd, d = o % hd;
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp) {
      acc_s[i][sp] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
          pr, static_cast<uint32_t>(((h * a.max_splits + sp) * rec + d) * 4), 0, 0));
    }
  }
  // (max, sum) of (head tid / MAXS, split tid % MAXS); past the last head the
  // offsets leave the buffer and read 0.
  const uint32_t ml = static_cast<uint32_t>(
      (((tid / MAXS) * a.max_splits + tid % MAXS) * rec + hd) * 4);
  const float mv = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(pr, ml, 0, 0));
  const float lv = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(pr, ml + 4u, 0, 0));
  __builtin_amdgcn_sched_barrier(0);  // every load is in flight
  const int pos = min(*a.pos, a.max_seq - 1);
  const int splits = pos / a.span + 1;
  if (tid < a.heads * MAXS) {
    ms[tid / MAXS][tid % MAXS] = mv;
    ls[tid / MAXS][tid % MAXS] = lv;
  }
  __syncthreads();
  if (tid < a.heads) {
    float mm = ms[tid][0];
#pragma unroll
    for (int sp = 1; sp < MAXS; ++sp) {
      if (sp < splits) mm = fmaxf(mm, ms[tid][sp]);
    }
    float e[MAXS], ll = 0.0f;
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp) {
      e[sp] = sp < splits ? exp_nonpos_fast(ms[tid][sp] - mm) : 0.0f;
      if (sp < splits) ll = fmaf(ls[tid][sp], e[sp], ll);
    }
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp) hw[tid][sp] = e[sp] / ll;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int o = tid + kBlock * i;
    if (o < a.k) {
      const int h = o / hd;
      float v = 0.0f;
#pragma unroll
      for (int sp = 0; sp < MAXS; ++sp) {
        if (sp < splits) v = fmaf(acc_s[i][sp], hw[h][sp], v);
      }
      attn[o] = bf16_to_f32(f32_to_bf16(v));  // the attention output is BF16
    }
  }
  __syncthreads();
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int i = 0; i < SLABS; ++i) {
    const int c = i * kWave + lane;
    float xv[kChunk];
#pragma unroll
    for (int e = 0; e < kChunk; ++e) xv[e] = c < chunks ? attn[kChunk * c + e] : 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (W8) {
        acc[r] = fmaf(dot16_i8(wq[r][i], reinterpret_cast<const float(&)[16]>(xv)),
                      bf16_to_f32(sc[r][i]), acc[r]);
      } else {
        acc[r] = dot8_bf16(wq[r][i], reinterpret_cast<const float(&)[8]>(xv), acc[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = wave_sum(acc[r]);
    const int row = row0 + r;
    // (x[row] is read here, not with the weights: requested up front it
    // measured 0.1 us slower)
    if (lane == 0 && row < a.n) gstore(a.x + row, f32_to_bf16(v + bf16_to_f32(gload(a.x + row))));
  }
}

// ------------------------------------------------------------ launchers --

// int8 rows: up to 8 slabs of 1024 weights (K <= 8192); BF16 rows: up to 10
// slabs of 512 (K <= 5120, the 4864 of the Qwen2.5-0.5B down projection
// included).
bool gemv_rows_supported(int k, bool w8) {
  return k >= 64 && k % 64 == 0 && k <= (w8 ? 8 * 1024 : 10 * 512);
}

template <class F, int MAXS>
static void launch_gemv_rows_fmt(const GemvRowsArgs& a, hipStream_t stream) {
  const dim3 grid((a.n + kWaves - 1) / kWaves), block(kBlock);
  switch (fused_slabs(a.k, F::C == W8Fmt::C)) {
#define QLIN_ROWS(S)                                                                    \
  case S:                                                                               \
    hipLaunchKernelGGL((gemv_rows_kernel<F, S>), grid, block, 0, stream, a);            \
    break;
    QLIN_ROWS(1)
    QLIN_ROWS(2)
    QLIN_ROWS(3)
    QLIN_ROWS(4)
    QLIN_ROWS(5)
    QLIN_ROWS(6)
    QLIN_ROWS(7)
    QLIN_ROWS(8)
    QLIN_ROWS(9)
    default:
      hipLaunchKernelGGL((gemv_rows_kernel<F, MAXS>), grid, block, 0, stream, a);
      break;
#undef QLIN_ROWS
  }
}

void launch_gemv_rows(const GemvRowsArgs& a, bool w8, hipStream_t stream) {
  if (w8) {
    launch_gemv_rows_fmt<W8Fmt, 8>(a, stream);
  } else {
    launch_gemv_rows_fmt<Bf16Fmt, 10>(a, stream);
  }
}

int norm_gemv_slabs(int k, bool w8) { return fused_slabs(k, w8); }

int norm_qkv_rope_blocks(int heads, int kv_heads, int head_dim) {
  const int tasks = (heads + 2 * kv_heads) * (head_dim / 2);
  return (tasks + kWaves - 1) / kWaves;
}

bool norm_gemv_supported(int k, bool w8) {
  return k >= 64 && k % 64 == 0 && norm_gemv_slabs(k, w8) <= kNormGemvMaxSlabs;
}

bool norm_qkv_rope_supported(int k, int head_dim, bool w8) {
  return norm_gemv_supported(k, w8) && head_dim % 2 == 0 && head_dim >= 2;
}

template <class F>
static void launch_norm_qkv_rope_fmt(const QkvRopeArgs& a, hipStream_t stream) {
  const dim3 grid(norm_qkv_rope_blocks(a.heads, a.kv_heads, a.head_dim)), block(kBlock);
  switch (fused_slabs(a.k, F::C == W8Fmt::C)) {
    case 1:
      hipLaunchKernelGGL((norm_qkv_rope_kernel<F, 1>), grid, block, 0, stream, a);
      break;
    case 2:
      hipLaunchKernelGGL((norm_qkv_rope_kernel<F, 2>), grid, block, 0, stream, a);
      break;
    default:
      hipLaunchKernelGGL((norm_qkv_rope_kernel<F, 4>), grid, block, 0, stream, a);
      break;
  }
}

void launch_norm_qkv_rope(const QkvRopeArgs& a, bool w8, hipStream_t stream) {
  if (w8) {
    launch_norm_qkv_rope_fmt<W8Fmt>(a, stream);
  } else {
    launch_norm_qkv_rope_fmt<Bf16Fmt>(a, stream);
  }
}

int norm_gemv_blocks(int n, int rows_per_wave) {
  const int rows = kWaves * rows_per_wave;
  return (n + rows - 1) / rows;
}

template <class F, int SLABS, bool PAIR>
static void launch_norm_gemv_rows(const NormGemvArgs& a, int blocks, hipStream_t stream) {
  switch (a.rows_per_wave) {
    case 4:
      hipLaunchKernelGGL((norm_gemv_kernel<F, SLABS, PAIR, 4>), dim3(blocks), dim3(kBlock), 0,
                         stream, a);
      break;
    case 2:
      hipLaunchKernelGGL((norm_gemv_kernel<F, SLABS, PAIR, 2>), dim3(blocks), dim3(kBlock), 0,
                         stream, a);
      break;
    default:
      hipLaunchKernelGGL((norm_gemv_kernel<F, SLABS, PAIR, 1>), dim3(blocks), dim3(kBlock), 0,
                         stream, a);
      break;
  }
}

template <class F, bool PAIR>
static void launch_norm_gemv_fmt(const NormGemvArgs& a, int blocks, hipStream_t stream) {
  switch (fused_slabs(a.k, F::C == W8Fmt::C)) {
    case 1:
      launch_norm_gemv_rows<F, 1, PAIR>(a, blocks, stream);
      break;
    case 2:
      launch_norm_gemv_rows<F, 2, PAIR>(a, blocks, stream);
      break;
    default:
      launch_norm_gemv_rows<F, 4, PAIR>(a, blocks, stream);
      break;
  }
}

void launch_norm_gemv(const NormGemvArgs& a, int blocks, bool pair, bool w8,
                      hipStream_t stream) {
  if (w8) {
    if (pair) {
      launch_norm_gemv_fmt<W8Fmt, true>(a, blocks, stream);
    } else {
      launch_norm_gemv_fmt<W8Fmt, false>(a, blocks, stream);
    }
  } else {
    if (pair) {
      launch_norm_gemv_fmt<Bf16Fmt, true>(a, blocks, stream);
    } else {
      launch_norm_gemv_fmt<Bf16Fmt, false>(a, blocks, stream);
    }
  }
}

int attn_o_slabs(int k, bool w8) {
  const int per_slab = kWave * (w8 ? 16 : 8);
  const int slabs = (k + per_slab - 1) / per_slab;
  return slabs <= 1 ? 1 : slabs <= 2 ? 2 : slabs <= 4 ? 4 : 8;
}

bool attn_o_supported(int k, int heads, bool w8) {
  const int chunk = w8 ? 16 : 8;
  return k % (w8 ? 64 : 8) == 0 && k % chunk == 0 && heads <= kAttnOMaxHeads &&
         attn_o_slabs(k, w8) <= (w8 ? 4 : 8) && heads * kAttnMaxSplits <= kBlock;
}

// Output rows per wave of the o-projection.  Each workgroup merges every
// head's partials, so wider workgroups repeat that merge less often, but
// measured at context 768 one row per wave (224 workgroups) is fastest:
// 5.22 us against 5.79 (2 rows) and 6.40 (4 rows).
constexpr int kAttnORowsPerWave = 1;

template <int SLABS, bool W8>
static void launch_attn_o_slabs(const AttnOArgs& a, hipStream_t stream) {
  constexpr int R = kAttnORowsPerWave;
  const dim3 grid((a.n + kWaves * R - 1) / (kWaves * R)), block(kBlock);
  if (a.max_splits <= 1) {
    hipLaunchKernelGGL((attn_o_gemv_kernel<SLABS, W8, 1, R>), grid, block, 0, stream, a);
  } else if (a.max_splits <= 2) {
    hipLaunchKernelGGL((attn_o_gemv_kernel<SLABS, W8, 2, R>), grid, block, 0, stream, a);
  } else if (a.max_splits <= 4) {
    hipLaunchKernelGGL((attn_o_gemv_kernel<SLABS, W8, 4, R>), grid, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL((attn_o_gemv_kernel<SLABS, W8, 8, R>), grid, block, 0, stream, a);
  }
}

void launch_attn_o_gemv(const AttnOArgs& a, bool w8, hipStream_t stream) {
  const int slabs = attn_o_slabs(a.k, w8);
  if (w8) {
    if (slabs == 1) {
      launch_attn_o_slabs<1, true>(a, stream);
    } else if (slabs == 2) {
      launch_attn_o_slabs<2, true>(a, stream);
    } else {
      launch_attn_o_slabs<4, true>(a, stream);
    }
  } else {
    if (slabs <= 2) {
      launch_attn_o_slabs<2, false>(a, stream);
    } else if (slabs == 4) {
      launch_attn_o_slabs<4, false>(a, stream);
    } else {
      launch_attn_o_slabs<8, false>(a, stream);
    }
  }
}

int lm_head_decode_slabs(int k) { return (k + 511) / 512; }

bool lm_head_decode_supported(int k) {
  return k >= 8 && k % 8 == 0 && lm_head_decode_slabs(k) <= kLmHeadMaxSlabs;
}

int lm_head_decode_blocks(int vocab) {
  // Two workgroups per CU on 256 CUs (the best of a sweep over 256-8192
  // workgroups and 1, 2 or 4 rows per task at V = 151936, K = 896: every
  // workgroup also takes the finishing counter once, so more of them cost
  // more); fewer for small vocabularies (at least one task per wave).
  const int cap = 512;
  const int need = (vocab + kWaves * kLmHeadRows - 1) / (kWaves * kLmHeadRows);
  return need < cap ? need : cap;
}

// A wave keeps two tasks of R rows x SLABS 16-byte chunks in flight (the
// current one and the next), 8 VGPRs per (row, chunk): R x SLABS is capped at
// 16 so that they fit without spilling (K > 2048 takes fewer rows per task).
template <int SLABS, int R>
static void launch_lm_head_fit(const LmHeadDecodeArgs& a, int grid, hipStream_t stream) {
  constexpr int kFit = R * SLABS > 16 ? 16 / SLABS : R;
  hipLaunchKernelGGL((lm_head_decode_kernel<SLABS, kFit>), dim3(grid), dim3(kBlock), 0, stream,
                     a);
}

template <int R>
static void launch_lm_head_rows(const LmHeadDecodeArgs& a, int grid, hipStream_t stream) {
  switch (lm_head_decode_slabs(a.k)) {
    case 1:
      launch_lm_head_fit<1, R>(a, grid, stream);
      break;
    case 2:
      launch_lm_head_fit<2, R>(a, grid, stream);
      break;
    case 3:
    case 4:
      launch_lm_head_fit<4, R>(a, grid, stream);
      break;
    default:
      launch_lm_head_fit<8, R>(a, grid, stream);
      break;
  }
}

void launch_lm_head_decode_shape(const LmHeadDecodeArgs& a, int grid, int rows,
                                 hipStream_t stream) {
  if (rows == 8) {
    launch_lm_head_rows<8>(a, grid, stream);
  } else if (rows == 4) {
    launch_lm_head_rows<4>(a, grid, stream);
  } else if (rows == 1) {
    launch_lm_head_rows<1>(a, grid, stream);
  } else {
    launch_lm_head_rows<2>(a, grid, stream);
  }
}

void launch_lm_head_decode(const LmHeadDecodeArgs& a, hipStream_t stream) {
  launch_lm_head_decode_shape(a, lm_head_decode_blocks(a.vocab), kLmHeadRows, stream);
}

}  // namespace qlin
