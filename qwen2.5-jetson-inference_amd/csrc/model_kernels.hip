// Non-Linear kernels of the Qwen2 decode step and prefill for gfx950: token
// embedding, RMSNorm, RoPE with the KV-cache store, attention (decode split
// over the context with an in-kernel combine, causal prefill), SiLU-mul and
// the residual add.
//
// The decode kernels read the position and the current token from device
// memory (ModelState), so one decode step is a fixed sequence of launches
// that a HIP graph replays for every token with no host round trip.
//
// Reference behaviour restated (src/cuda/kernels.cu and src/cpu_ops.cpp):
//   embedding 18-62; rms_norm 64-116 (FP32 sum of squares, BF16 output);
//   rope 119-137 (rotate-half; here the cos/sin of each (position, pair)
//   come from a table the host fills with the CPU path's own float
//   arithmetic, cpu_ops.cpp:38-41); store_kv 139-157 (cache layout
//   [kv_head][max_seq][head_dim]); attention decode 159-218 and prefill
//   221-283 (softmax(q k / sqrt(d)) v, GQA head h -> kv head h / group);
//   add 285-300; silu_mul 302-324 (gate / (1 + exp(-gate)) * up).
#include <float.h>
#include <stdint.h>

#include "device_common.hpp"
#include "model_kernels.hpp"

namespace qlin {

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float load_bf16(const uint16_t* p) { return bf16_to_f32(*p); }

}  // namespace

// ------------------------------------------------------------ embedding --

// out[t] = table[tokens[t]] for t < count (rows of `hidden` BF16 words,
// copied as 16-byte chunks when hidden % 8 == 0).  Tokens are clamped into
// the table (the host validates prompt tokens; decode tokens come from the
// argmax, always in range).
__global__ __launch_bounds__(kThreads) void embedding_kernel(const uint16_t* __restrict__ table,
                                                             const int* __restrict__ tokens,
                                                             int count, int vocab, int hidden,
                                                             uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  if (t >= count) return;
  const int token = min(max(tokens[t], 0), vocab - 1);
  const uint16_t* src = table + static_cast<size_t>(token) * hidden;
  uint16_t* dst = out + static_cast<size_t>(t) * hidden;
  if ((hidden & 7) == 0) {
    for (int c = threadIdx.x; c < hidden / 8; c += kThreads) {
      reinterpret_cast<uint4*>(dst)[c] = reinterpret_cast<const uint4*>(src)[c];
    }
  } else {
    for (int c = threadIdx.x; c < hidden; c += kThreads) dst[c] = src[c];
  }
}

// --------------------------------------------------------------- RMSNorm --

// One block per row: out = bf16(x * scale * w), scale = 1 / sqrt(mean(x^2)
// + eps) with an FP32 sum of squares.
__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ w,
                                                            uint16_t* __restrict__ out, int rows,
                                                            int hidden, float eps) {
  const int row = blockIdx.x;
  if (row >= rows) return;
  const uint16_t* xr = x + static_cast<size_t>(row) * hidden;
  uint16_t* orow = out + static_cast<size_t>(row) * hidden;
  float sum = 0.0f;
  for (int i = threadIdx.x; i < hidden; i += kThreads) {
    const float v = load_bf16(xr + i);
    sum = fmaf(v, v, sum);
  }
  __shared__ float part[kThreads / kWave];
  sum = wave_sum(sum);
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = sum;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kThreads / kWave; ++i) total += part[i];
  const float scale = 1.0f / sqrtf(total / hidden + eps);
  for (int i = threadIdx.x; i < hidden; i += kThreads) {
    orow[i] = f32_to_bf16(load_bf16(xr + i) * scale * load_bf16(w + i));
  }
}

// Residual add and the RMSNorm behind it, one block per row: x = bf16(x +
// y) in place, then out = bf16(x * scale * w) of the new x (the two kernels'
// arithmetic and summation order, in one launch).  hidden <= 16 * kThreads.
__global__ __launch_bounds__(kThreads) void add_rms_norm_kernel(uint16_t* __restrict__ x,
                                                                const uint16_t* __restrict__ y,
                                                                const uint16_t* __restrict__ w,
                                                                uint16_t* __restrict__ out,
                                                                int rows, int hidden, float eps) {
  constexpr int kPer = 16;
  const int row = blockIdx.x;
  if (row >= rows) return;
  uint16_t* xr = x + static_cast<size_t>(row) * hidden;
  const uint16_t* yr = y + static_cast<size_t>(row) * hidden;
  uint16_t* orow = out + static_cast<size_t>(row) * hidden;
  float v[kPer];
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = threadIdx.x + j * kThreads;
    v[j] = 0.0f;
    if (i < hidden) {
      const uint16_t s = f32_to_bf16(load_bf16(xr + i) + load_bf16(yr + i));
      xr[i] = s;
      v[j] = bf16_to_f32(s);
      sum = fmaf(v[j], v[j], sum);
    }
  }
  __shared__ float part[kThreads / kWave];
  sum = wave_sum(sum);
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = sum;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kThreads / kWave; ++i) total += part[i];
  const float scale = 1.0f / sqrtf(total / hidden + eps);
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int i = threadIdx.x + j * kThreads;
    if (i < hidden) orow[i] = f32_to_bf16(v[j] * scale * load_bf16(w + i));
  }
}

// RMSNorm rows (with ADD: after the residual add x = bf16(x + y), in place),
// one wave per row and four rows per block: lane l takes the 8-element
// chunks l, l + 64, ... of the row with 16-byte loads and stores, and the
// sum of squares is reduced across the wave (DPP/permlane) with no LDS or
// barrier.  The elementwise arithmetic is rms_norm_kernel's and
// add_rms_norm_kernel's; the sum of squares is added in another order.
// With G (the prefill's first launch) the row is gathered from the
// embedding table (row tokens[row], clamped as embedding_kernel does),
// stored into x and normalized: the embedding and the first RMSNorm in one
// launch.
// hidden % 8 == 0, hidden <= 512 * CH, 16-byte aligned rows.
template <int CH, bool ADD, bool G>
__global__ __launch_bounds__(kThreads) void norm_rows_kernel(uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ y,
                                                             const uint16_t* __restrict__ w,
                                                             uint16_t* __restrict__ out,
                                                             int rows, int hidden, float eps,
                                                             const uint16_t* __restrict__ table,
                                                             const int* __restrict__ tokens,
                                                             int vocab) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
  if (row >= rows) return;  // the whole wave
  const int chunks = hidden >> 3;
  uint4* xr = reinterpret_cast<uint4*>(x + static_cast<size_t>(row) * hidden);
  const uint4* src = xr;
  if (G) {
    const int token = min(max(tokens[row], 0), vocab - 1);
    src = reinterpret_cast<const uint4*>(table + static_cast<size_t>(token) * hidden);
  }
  const uint4* yr = ADD ? reinterpret_cast<const uint4*>(y + static_cast<size_t>(row) * hidden)
                        : nullptr;
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  uint4* orow = reinterpret_cast<uint4*>(out + static_cast<size_t>(row) * hidden);
  uint4 xa[CH], ya[CH], wa[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {  // every load in flight at once (clamped, masked below)
    const int i = min(lane + kWave * c, chunks - 1);
    xa[c] = load_global16(src + i);
    if (ADD) ya[c] = load_global16(yr + i);
    wa[c] = load_global16(wr + i);
  }
  float v[CH][8];
  float sum = 0.0f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const bool live = lane + kWave * c < chunks;
    const uint32_t xs[4] = {xa[c].x, xa[c].y, xa[c].z, xa[c].w};
    const uint32_t ys[4] = {ADD ? ya[c].x : 0u, ADD ? ya[c].y : 0u, ADD ? ya[c].z : 0u,
                            ADD ? ya[c].w : 0u};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float a0 = bf16_lo(xs[e]), a1 = bf16_hi(xs[e]);
      if (ADD) {
        a0 = bf16_to_f32(f32_to_bf16(a0 + bf16_lo(ys[e])));
        a1 = bf16_to_f32(f32_to_bf16(a1 + bf16_hi(ys[e])));
      }
      v[c][2 * e] = a0;
      v[c][2 * e + 1] = a1;
      if (live) sum = fmaf(a1, a1, fmaf(a0, a0, sum));
    }
    if ((ADD || G) && live) {
      store_global16(xr + lane + kWave * c, make_uint4(pack2_bf16(v[c][0], v[c][1]),
                                                       pack2_bf16(v[c][2], v[c][3]),
                                                       pack2_bf16(v[c][4], v[c][5]),
                                                       pack2_bf16(v[c][6], v[c][7])));
    }
  }
  sum = wave_sum(sum);
  const float scale = 1.0f / sqrtf(sum / hidden + eps);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    if (lane + kWave * c >= chunks) continue;
    const uint32_t ws[4] = {wa[c].x, wa[c].y, wa[c].z, wa[c].w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = pack2_bf16(v[c][2 * e] * scale * bf16_lo(ws[e]),
                        v[c][2 * e + 1] * scale * bf16_hi(ws[e]));
    }
    store_global16(orow + lane + kWave * c, make_uint4(o[0], o[1], o[2], o[3]));
  }
}

// The wave-per-row form applies (16-byte aligned rows of whole chunks);
// chunks per lane for it, 0 if it does not.
int norm_rows_chunks(const void* x, const void* y, const void* w, const void* out, int hidden) {
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (hidden <= 0 || hidden % 8 != 0 || !a16(x) || (y && !a16(y)) || !a16(w) || !a16(out)) {
    return 0;
  }
  const int per = (hidden / 8 + kWave - 1) / kWave;
  return per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : per <= 8 ? 8 : 0;
}

template <bool ADD, bool GATHER = false>
void launch_norm_rows(int ch, uint16_t* x, const uint16_t* y, const uint16_t* w, uint16_t* out,
                      int rows, int hidden, float eps, hipStream_t stream,
                      const uint16_t* table = nullptr, const int* tokens = nullptr,
                      int vocab = 0) {
  const dim3 grid((rows + kThreads / kWave - 1) / (kThreads / kWave)), block(kThreads);
  constexpr bool G = !ADD && GATHER;
  switch (ch) {
    case 1:
      hipLaunchKernelGGL((norm_rows_kernel<1, ADD, G>), grid, block, 0, stream, x, y, w, out,
                         rows, hidden, eps, table, tokens, vocab);
      break;
    case 2:
      hipLaunchKernelGGL((norm_rows_kernel<2, ADD, G>), grid, block, 0, stream, x, y, w, out,
                         rows, hidden, eps, table, tokens, vocab);
      break;
    case 4:
      hipLaunchKernelGGL((norm_rows_kernel<4, ADD, G>), grid, block, 0, stream, x, y, w, out,
                         rows, hidden, eps, table, tokens, vocab);
      break;
    default:
      hipLaunchKernelGGL((norm_rows_kernel<8, ADD, G>), grid, block, 0, stream, x, y, w, out,
                         rows, hidden, eps, table, tokens, vocab);
      break;
  }
}

// ------------------------------------------------------- RoPE + KV store --


// Prefill: tokens t < count at positions start + t.  q [count][heads][d]
// and k [count][kv_heads][d] are rotated in place (BF16 rounding, as the
// reference's rope kernel stores BF16); k and v are copied into the caches.
// One block per token; thread j of the block handles pair j % half of head
// j / half.
__global__ __launch_bounds__(kThreads) void rope_store_kernel(
    uint16_t* __restrict__ q, uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    uint16_t* __restrict__ key_cache, uint16_t* __restrict__ value_cache,
    const float2* __restrict__ rope, int count, int start, int heads, int kv_heads,
    int head_dim, int max_seq) {
  const int t = blockIdx.x;
  const int pos = start + t;
  if (t >= count || pos >= max_seq) return;
  const int half = head_dim / 2;
  const float2* cs = rope + static_cast<size_t>(pos) * half;
  for (int j = threadIdx.x; j < (heads + kv_heads) * half; j += kThreads) {
    const int head = j / half, i = j % half;
    uint16_t* base = head < heads
                         ? q + (static_cast<size_t>(t) * heads + head) * head_dim
                         : k + (static_cast<size_t>(t) * kv_heads + head - heads) * head_dim;
    float a = load_bf16(base + i), b = load_bf16(base + i + half);
    rope_pair(a, b, cs[i]);
    base[i] = f32_to_bf16(a);
    base[i + half] = f32_to_bf16(b);
  }
  __syncthreads();  // the rotated k of this token is complete
  for (int j = threadIdx.x; j < kv_heads * head_dim; j += kThreads) {
    const int g = j / head_dim, d = j % head_dim;
    const size_t at = (static_cast<size_t>(g) * max_seq + pos) * head_dim + d;
    key_cache[at] = k[(static_cast<size_t>(t) * kv_heads + g) * head_dim + d];
    value_cache[at] = v[(static_cast<size_t>(t) * kv_heads + g) * head_dim + d];
  }
}

// The same, one wave per token and four tokens per block, with 16-byte
// accesses: a unit is chunk c (8 dimensions) of the first half of a q or k
// head and its rotation partner, chunk c + half / 8, so a lane loads both,
// rotates its 8 pairs (rope_pair, as rope_store_kernel) and stores both; a
// k head's rotated chunks go to the key cache from the same registers, and
// v's chunks are copied to the value cache 16 bytes at a time.  head_dim % 16
// == 0 and 16-byte aligned tensors.
__global__ __launch_bounds__(kThreads) void rope_store_rows_kernel(
    uint16_t* __restrict__ q, uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    uint16_t* __restrict__ key_cache, uint16_t* __restrict__ value_cache,
    const float2* __restrict__ rope, int count, int start, int heads, int kv_heads,
    int head_dim, int max_seq) {
  const int lane = threadIdx.x & (kWave - 1);
  const int t = blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
  const int pos = start + t;
  if (t >= count || pos >= max_seq) return;  // the whole wave
  const int half_chunks = head_dim / 16;     // chunks in half a head
  const int units = (heads + kv_heads) * half_chunks;
  const float2* cs = rope + static_cast<size_t>(pos) * (head_dim / 2);
  for (int u = lane; u < units; u += kWave) {
    const int head = u / half_chunks, c = u % half_chunks;
    const bool is_k = head >= heads;
    uint16_t* base = is_k ? k + (static_cast<size_t>(t) * kv_heads + head - heads) * head_dim
                          : q + (static_cast<size_t>(t) * heads + head) * head_dim;
    const uint4 lo = load_global16(base + 8 * c);
    const uint4 hi = load_global16(base + head_dim / 2 + 8 * c);
    float2 r[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 two = *reinterpret_cast<const float4*>(cs + 8 * c + 2 * j);
      r[2 * j] = make_float2(two.x, two.y);
      r[2 * j + 1] = make_float2(two.z, two.w);
    }
    const uint32_t l4[4] = {lo.x, lo.y, lo.z, lo.w}, h4[4] = {hi.x, hi.y, hi.z, hi.w};
    uint32_t ol[4], oh[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float a0 = bf16_lo(l4[e]), b0 = bf16_lo(h4[e]);
      float a1 = bf16_hi(l4[e]), b1 = bf16_hi(h4[e]);
      rope_pair(a0, b0, r[2 * e]);
      rope_pair(a1, b1, r[2 * e + 1]);
      ol[e] = pack2_bf16(a0, a1);
      oh[e] = pack2_bf16(b0, b1);
    }
    const uint4 nl = make_uint4(ol[0], ol[1], ol[2], ol[3]);
    const uint4 nh = make_uint4(oh[0], oh[1], oh[2], oh[3]);
    store_global16(base + 8 * c, nl);
    store_global16(base + head_dim / 2 + 8 * c, nh);
    if (is_k) {
      uint16_t* row =
          key_cache + (static_cast<size_t>(head - heads) * max_seq + pos) * head_dim;
      store_global16(row + 8 * c, nl);
      store_global16(row + head_dim / 2 + 8 * c, nh);
    }
  }
  const int v_chunks = kv_heads * head_dim / 8;
  for (int u = lane; u < v_chunks; u += kWave) {
    const int g = u / (head_dim / 8), c = u % (head_dim / 8);
    const uint4 val =
        load_global16(v + (static_cast<size_t>(t) * kv_heads + g) * head_dim + 8 * c);
    store_global16(value_cache + (static_cast<size_t>(g) * max_seq + pos) * head_dim + 8 * c,
                   val);
  }
}

// ------------------------------------------------------ decode attention --

// One decode step's attention over the context [0, pos] of query head h
// (kv head g = h / group), in one of two forms:
//  - whole (HD = 64, max_seq <= kAttnWholeMax): one workgroup per query
//    head over the whole context, writing the head's normalised output
//    bf16(sum p v / sum p) (attention_decode_whole_kernel below); the
//    o-projection is then a plain GEMV on it.
//  - split: workgroup (c, h) takes the positions [c span, (c + 1) span)
//    with kAttnWaves waves and stores the span's (acc[HD], max, sum)
//    partial at partial[(h * max_splits + c) * (HD + 2)]; the o-projection
//    kernel merges the partials of the ceil((pos + 1) / span) spans
//    (attn_o_gemv_kernel).  This keeps long contexts spread over many CUs.
// In a tile lane p holds position p's key and value rows (16-byte buffer
// loads whose range ends at the context, so rows past it read as zeros
// without a branch around the loads), scores it against the rotated q (in
// LDS), and the tile's value rows go through the wave's LDS slice so that
// lane d can accumulate output dimension d (and d + 64 when HD = 128).
// The softmax runs online across a wave's tiles.  The query heads of a kv
// head read the same rows; they meet in L2 or the memory-side cache.
//
// Latency: a wave's first tile is requested at kernel entry, before the q
// rotation, and (HD = 64) each next tile before the current one is
// computed.
//
// Position pos is the new token: its k (rotated here) and v come from
// k_new / v_new through LDS, never from the cache, and the workgroup of
// the first query head of the kv head whose span holds pos writes them into
// the caches.
constexpr int kTile = 64;

template <int HD>
__device__ __forceinline__ void load_tile_rows(__amdgpu_buffer_rsrc_t kr_rsrc,
                                               __amdgpu_buffer_rsrc_t vr_rsrc, int p,
                                               uint4 (&kr)[HD / 8], uint4 (&vr)[HD / 8]) {
  const uint32_t row = static_cast<uint32_t>(p) * HD * 2u;
#pragma unroll
  for (int j = 0; j < HD / 8; ++j) {
    kr[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kr_rsrc, row + 16u * j,
                                                                            0, 0));
  }
#pragma unroll
  for (int j = 0; j < HD / 8; ++j) {
    vr[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vr_rsrc, row + 16u * j,
                                                                            0, 0));
  }
}

// ROPED: q is rotated already and the caches hold the token's k and v at
// pos (the attention_decode_bf16 contract); otherwise q and k_new are
// rotated here and the token's k and v stored (the model's decode step).
template <int HD, bool ROPED>
__global__ __launch_bounds__(kAttnWaves * kWave) void attention_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_new,
    const uint16_t* __restrict__ v_new, uint16_t* __restrict__ key_cache,
    uint16_t* __restrict__ value_cache, const float2* __restrict__ rope,
    const int* __restrict__ pos_ptr, int heads, int kv_heads, int max_seq, int span,
    int max_splits, float* __restrict__ partial) {
  constexpr int W = kAttnWaves;
  constexpr int half = HD / 2;
  constexpr int kDims = HD / kWave;  // output dimensions per lane
  constexpr int kPieces = HD / 8;    // 16-byte pieces per row
  constexpr int kRow = HD + 8;       // LDS row stride (BF16 elements), padded
  constexpr bool kPrefetch = HD <= 64;  // register budget
  const int c = blockIdx.x;
  const int h = blockIdx.y;
  const int pos = min(*pos_ptr, max_seq - 1);
  const int seq = pos + 1;
  const int begin = c * span;
  if (begin >= seq) return;  // the grid covers max_seq; spans past the context exit
  const int end = min(seq, begin + span);
  const int group = heads / kv_heads;
  const int g = h / group;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const size_t head_base = static_cast<size_t>(g) * max_seq * HD;
  const __amdgpu_buffer_rsrc_t kr_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(key_cache + head_base, 0, end * HD * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t vr_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(value_cache + head_base, 0, end * HD * 2, 0x00020000);

  uint4 kr[kPieces], vr[kPieces];
  load_tile_rows<HD>(kr_rsrc, vr_rsrc, begin + wave * kTile + lane, kr, vr);

  __shared__ float qs[HD];
  __shared__ __align__(16) uint16_t knew[HD];
  __shared__ __align__(16) uint16_t vnew[HD];
  __shared__ __align__(16) uint16_t vt[W][kTile][kRow];
  __shared__ float et[W][kTile];
  __shared__ float wm[W], wl[W];
  __shared__ float wacc[W][HD];

  // q of head h and this token's k, rotated and rounded to BF16 (as the
  // reference's rope kernel stores them), and this token's v.
  if (ROPED) {
    if (tid < HD) qs[tid] = load_bf16(q + static_cast<size_t>(h) * HD + tid);
  } else if (tid < half) {
    const float2* cs = rope + static_cast<size_t>(pos) * half;
    const uint16_t* qh = q + static_cast<size_t>(h) * HD;
    const uint16_t* kh = k_new + static_cast<size_t>(g) * HD;
    const float2 r = cs[tid];
    float q0 = load_bf16(qh + tid), q1 = load_bf16(qh + tid + half);
    float k0 = load_bf16(kh + tid), k1 = load_bf16(kh + tid + half);
    rope_pair(q0, q1, r);
    rope_pair(k0, k1, r);
    qs[tid] = bf16_to_f32(f32_to_bf16(q0));
    qs[tid + half] = bf16_to_f32(f32_to_bf16(q1));
    knew[tid] = f32_to_bf16(k0);
    knew[tid + half] = f32_to_bf16(k1);
  } else if (tid < half + kPieces) {
    const int j = tid - half;
    reinterpret_cast<uint4*>(vnew)[j] =
        reinterpret_cast<const uint4*>(v_new + static_cast<size_t>(g) * HD)[j];
  }
  __syncthreads();
  if (!ROPED && h % group == 0 && pos >= begin && pos < end && tid < 2 * kPieces) {
    // The kv head's first query head, in the span holding pos, stores the
    // new token's k and v.
    const int j = tid % kPieces;
    uint16_t* dst = (tid < kPieces ? key_cache : value_cache) + head_base +
                    static_cast<size_t>(pos) * HD;
    const uint16_t* src = tid < kPieces ? knew : vnew;
    reinterpret_cast<uint4*>(dst)[j] = reinterpret_cast<const uint4*>(src)[j];
  }

  const float scale = 1.0f / sqrtf(static_cast<float>(HD));
  float m = -INFINITY, l = 0.0f;
  float acc[kDims];
#pragma unroll
  for (int j = 0; j < kDims; ++j) acc[j] = 0.0f;
  for (int t0 = begin + wave * kTile; t0 < end; t0 += W * kTile) {
    const int p = t0 + lane;
    uint4 kn[kPieces], vn[kPieces];
    if (kPrefetch && t0 + W * kTile < end) {
      load_tile_rows<HD>(kr_rsrc, vr_rsrc, p + W * kTile, kn, vn);
    }
    if (!ROPED && p == pos) {
#pragma unroll
      for (int j = 0; j < kPieces; ++j) {
        kr[j] = reinterpret_cast<const uint4*>(knew)[j];
        vr[j] = reinterpret_cast<const uint4*>(vnew)[j];
      }
    }
    const bool valid = p < end;
    float dot = 0.0f;
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
      dot = fmaf(qs[8 * j + 0], bf16_lo(kr[j].x), dot);
      dot = fmaf(qs[8 * j + 1], bf16_hi(kr[j].x), dot);
      dot = fmaf(qs[8 * j + 2], bf16_lo(kr[j].y), dot);
      dot = fmaf(qs[8 * j + 3], bf16_hi(kr[j].y), dot);
      dot = fmaf(qs[8 * j + 4], bf16_lo(kr[j].z), dot);
      dot = fmaf(qs[8 * j + 5], bf16_hi(kr[j].z), dot);
      dot = fmaf(qs[8 * j + 6], bf16_lo(kr[j].w), dot);
      dot = fmaf(qs[8 * j + 7], bf16_hi(kr[j].w), dot);
    }
    const float sc = valid ? dot * scale : -INFINITY;
    const float bm = wave_max(sc);
    const float nm = fmaxf(m, bm);
    const float e = valid ? exp_nonpos_fast(sc - nm) : 0.0f;
    const float f = exp_nonpos_fast(m - nm);  // m = -inf on a wave's first tile: f = 0
    l = fmaf(l, f, wave_sum(e));
#pragma unroll
    for (int j = 0; j < kDims; ++j) acc[j] *= f;
    m = nm;
    et[wave][lane] = e;
#pragma unroll
    for (int j = 0; j < kPieces; ++j) reinterpret_cast<uint4*>(vt[wave][lane])[j] = vr[j];
    __builtin_amdgcn_wave_barrier();  // the tile is in this wave's LDS slice
    const int n = min(kTile, end - t0);
#pragma unroll 8
    for (int pp = 0; pp < n; ++pp) {
      const float w = et[wave][pp];
#pragma unroll
      for (int j = 0; j < kDims; ++j) {
        acc[j] = fmaf(w, bf16_to_f32(vt[wave][pp][lane + kWave * j]), acc[j]);
      }
    }
    __builtin_amdgcn_wave_barrier();  // reads done before the next tile's writes
    if (kPrefetch) {
#pragma unroll
      for (int j = 0; j < kPieces; ++j) {
        kr[j] = kn[j];
        vr[j] = vn[j];
      }
    } else if (t0 + W * kTile < end) {
      load_tile_rows<HD>(kr_rsrc, vr_rsrc, p + W * kTile, kr, vr);
    }
  }
  if (lane == 0) {
    wm[wave] = m;
    wl[wave] = l;
  }
#pragma unroll
  for (int j = 0; j < kDims; ++j) wacc[wave][lane + kWave * j] = acc[j];
  __syncthreads();
  // Merge the waves (idle waves have l = 0) and store the span's partial.
  if (tid < HD) {
    float mm = wm[0];
#pragma unroll
    for (int w = 1; w < W; ++w) mm = fmaxf(mm, wm[w]);
    float ll = 0.0f, aa = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = wl[w] > 0.0f ? exp_nonpos_fast(wm[w] - mm) : 0.0f;
      ll = fmaf(wl[w], f, ll);
      aa = fmaf(wacc[w][tid], f, aa);
    }
    float* rec = partial + (static_cast<size_t>(h) * max_splits + c) * (HD + 2);
    rec[tid] = aa;
    if (tid == 0) {
      rec[HD] = mm;
      rec[HD + 1] = ll;
    }
  }
}

// The whole-context form at HD = 64: one workgroup of W waves per query
// head h, wave w taking the 64-position tiles w, w + W, ... of the context.
// Pre-rotated (the q|k|v launch rotated q and stored the token's k and v):
// the tiles cover [0, pos]; otherwise (q and the new k rotated here) the
// cached positions [0, pos).  8 waves of two tiles each up to
// kAttnWholeMax positions, both tiles requested at entry.
//  - Loads are coalesced: instruction j of a wave reads rows 8 j .. 8 j + 7
//    of its tile, 1 KiB contiguous, lane l taking row 8 j + l / 8 and its
//    16-byte piece l % 8 (dimensions 8 (l % 8) .. + 7).  (One row per lane
//    touches 64 cache lines per instruction and re-reads each 8 times,
//    which overflows the CU's L1 with every wave's rows in flight.)
//  - Each wave rotates q and the new k itself, lane l from its piece l % 8
//    and the rotation partner piece of lane l ^ 4: no barrier before the
//    tile loop.  These small loads are issued before the tile loads, so
//    waiting for them does not wait for the tiles.
//  - A row's score is the sum of its 8 lanes' partial dot products, taken
//    by a reduce-scatter in the 8-lane group (DPP) that leaves lane l with
//    the score of row 8 (l % 8) + l / 8.  Its softmax weight goes back to
//    the 8 lanes holding that row's value pieces (ds_swizzle broadcast),
//    each lane sums weight x value over its 8 rows for its 8 dimensions,
//    and a reduce-scatter over the 8 row groups (permlane swaps, DPP)
//    leaves lane l with dimension 8 (l % 8) + l / 8 of the wave's sum.
//  - The new token (position pos) is not read from the cache: its score
//    q . k_new and value v_new enter the merge as one more (max, sum, acc)
//    record.  The waves' records are merged in LDS and the workgroup writes
//    bf16(sum p v / sum p) to out[h * 64 + d].
constexpr int kWholeWaves = kAttnWholeMax / kTile / 2;

constexpr int kDppRowRor8 = 0x128;  // row_ror:8, lane i of a row of 16 reads lane i ^ 8

// Lane (l & ~7) | J of the lane's group of 8 (ds_swizzle, bit-mask mode).
template <int J>
__device__ __forceinline__ float group8_lane(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x18 | (J << 5)));
}

// Reduce-scatter of v[0..8) over the lane's group of 8: returns the group
// total of v[l % 8].  The first step pairs lane i with 7 - i (half-row
// mirror); they differ in bit 2, which picks the half each keeps.
__device__ __forceinline__ float group8_reduce_scatter(float (&v)[8], int lane) {
  {
    const bool up = (lane & 4) != 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float send = up ? v[i] : v[i + 4];
      const float keep = up ? v[i + 4] : v[i];
      v[i] = keep + dpp_from<kDppRowHalfMirror>(send);
    }
  }
  {
    const bool up = (lane & 2) != 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float send = up ? v[i] : v[i + 2];
      const float keep = up ? v[i + 2] : v[i];
      v[i] = keep + dpp_from<kDppQuadSwap2>(send);
    }
  }
  const bool up = (lane & 1) != 0;
  const float send = up ? v[0] : v[1];
  const float keep = up ? v[1] : v[0];
  return keep + dpp_from<kDppQuadSwap1>(send);
}

// Reduce-scatter of v[0..8) over the 8 lanes l % 8 + 8 g (g = 0..7):
// returns the total of v[l / 8] over those lanes.
__device__ __forceinline__ float rows8_reduce_scatter(float (&v)[8], int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = swap32_sum(v[i], v[i + 4]);
#pragma unroll
  for (int i = 0; i < 2; ++i) v[i] = swap16_sum(v[i], v[i + 2]);
  const bool up = (lane & 8) != 0;
  const float send = up ? v[0] : v[1];
  const float keep = up ? v[1] : v[0];
  return keep + dpp_from<kDppRowRor8>(send);
}

// Sum over 8 dimensions of q * k, both BF16 pairs packed in 32-bit words
// (v_dot2c_f32_bf16: the products are exact, FP32 accumulation).
__device__ __forceinline__ float dot8_packed_bf16(const uint32_t (&q)[4], const uint4 k) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  float d = 0.0f;
  d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q[0]),
                                      __builtin_bit_cast(bf16x2, k.x), d, false);
  d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q[1]),
                                      __builtin_bit_cast(bf16x2, k.y), d, false);
  d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q[2]),
                                      __builtin_bit_cast(bf16x2, k.z), d, false);
  d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, q[3]),
                                      __builtin_bit_cast(bf16x2, k.w), d, false);
  return d;
}

__device__ __forceinline__ void unpack8_bf16(const uint4 w, float (&o)[8]) {
  o[0] = bf16_lo(w.x); o[1] = bf16_hi(w.x); o[2] = bf16_lo(w.y); o[3] = bf16_hi(w.y);
  o[4] = bf16_lo(w.z); o[5] = bf16_hi(w.z); o[6] = bf16_lo(w.w); o[7] = bf16_hi(w.w);
}

// Workgroups of the whole-context attention.  Workgroup b runs on XCD
// b % kXcds (the dispatcher deals workgroups to the XCDs in turn), and each
// XCD has its own L2: the query heads that share a kv head are given
// workgroups of one XCD, so that kv head's cache rows come from HBM once and
// from that L2 for the others (with one workgroup per head in order, the
// seven heads of a kv head sat on seven XCDs and each fetched the rows from
// HBM: 9.4x the kernel's compulsory bytes).  Workgroups past the last kv
// head exit at once.
constexpr int kXcds = 8;

int whole_attention_blocks(int heads, int kv_heads) {
  return kXcds * ((kv_heads + kXcds - 1) / kXcds) * (heads / kv_heads);
}

// The query head of workgroup b, or -1 for a workgroup with none.
__device__ inline int whole_attention_head(int b, int heads, int kv_heads) {
  const int group = heads / kv_heads;
  const int x = b % kXcds, t = b / kXcds;
  const int g = (t / group) * kXcds + x;
  return g < kv_heads ? g * group + t % group : -1;
}

// The whole-context attention of a pre-rotated q over caches that hold the
// new token's k and v already (attention_decode_bf16, kernels.cu:400-490).
// Waves of the workgroup: kWholeWaves, two tiles each, both in flight.
// Measured at contexts 256-1023 (us per launch): 8 waves x 2 tiles
// 4.4-6.4, 16 x 1 4.3-8.3, 4 x 4 5.0-7.7.
__global__ __launch_bounds__(kWholeWaves * kWave) void attention_decode_whole_kernel(
    const uint16_t* __restrict__ q, uint16_t* __restrict__ key_cache,
    uint16_t* __restrict__ value_cache, const int* __restrict__ pos_ptr, int heads,
    int kv_heads, int max_seq, uint16_t* __restrict__ out) {
  constexpr int HD = 64, W = kWholeWaves;
  constexpr int kPieces = HD / 8;            // 16-byte pieces per row (8)
  constexpr int kRowsPer = kWave / kPieces;  // rows per load instruction (8)
  constexpr bool kPrefetch = true;           // a second tile per wave
  static_assert(W * kTile * 2 >= kAttnWholeMax, "tiles cover the context");
  const int h = whole_attention_head(blockIdx.x, heads, kv_heads);
  if (h < 0) return;
  const int group = heads / kv_heads;
  const int g = h / group;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int pc = lane % kPieces, rg = lane / kPieces;  // piece, row within instruction
  const size_t head_base = static_cast<size_t>(g) * max_seq * HD;
  const uint4* qh = reinterpret_cast<const uint4*>(q + static_cast<size_t>(h) * HD);
  const uint4 q_mine = qh[pc];
  // The tiles cover [0, pos] and go out before pos is known (rows past the
  // context are masked below).
  const int rows = max_seq;  // the cache rows the tiles may read
  __builtin_amdgcn_sched_barrier(0);  // the small loads go out before the tiles
  const __amdgpu_buffer_rsrc_t kr_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(key_cache + head_base, 0, rows * HD * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t vr_rsrc =
      __builtin_amdgcn_make_buffer_rsrc(value_cache + head_base, 0, rows * HD * 2, 0x00020000);
  auto load_tile = [&](int t0, __amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                       uint4 (&kr)[kPieces], uint4 (&vr)[kPieces]) {
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
      const uint32_t off = static_cast<uint32_t>((t0 + kRowsPer * j + rg) * HD * 2 + 16 * pc);
      kr[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, 0));
    }
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
      const uint32_t off = static_cast<uint32_t>((t0 + kRowsPer * j + rg) * HD * 2 + 16 * pc);
      vr[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, 0));
    }
  };
  uint4 kr[kPieces], vr[kPieces], kn[kPieces], vn[kPieces];
  load_tile(wave * kTile, kr_rsrc, vr_rsrc, kr, vr);
  const int pos = min(*pos_ptr, max_seq - 1);
  // Positions [0, end) come from the tiles.
  const int end = pos + 1;
  if (kPrefetch) {
    // The first tiles went out before the position arrived.  The second
    // tiles are bounded by the context: rows past it read as 0 without a
    // memory access (and are masked below), so the CU takes in only the
    // context's rows beyond the first W tiles.
    const uint32_t bytes = static_cast<uint32_t>(end) * HD * 2;
    load_tile((wave + W) * kTile,
              __builtin_amdgcn_make_buffer_rsrc(key_cache + head_base, 0, bytes, 0x00020000),
              __builtin_amdgcn_make_buffer_rsrc(value_cache + head_base, 0, bytes, 0x00020000),
              kn, vn);
  }

  const float scale = 1.0f / sqrtf(static_cast<float>(HD));
  const uint32_t qw[4] = {q_mine.x, q_mine.y, q_mine.z, q_mine.w};  // 8 q dimensions

  float m = -INFINITY, l = 0.0f;
  float acc8[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc8[t] = 0.0f;
  // One 64-position tile into the wave's online softmax (wave-uniform: a
  // tile past the context is skipped whole).
  auto tile = [&](int t0, const uint4 (&kt)[kPieces], const uint4 (&vt)[kPieces]) {
    if (t0 >= end) return;
    float part[kPieces];
#pragma unroll
    for (int j = 0; j < kPieces; ++j) part[j] = dot8_packed_bf16(qw, kt[j]);
    const float score = group8_reduce_scatter(part, lane);  // row 8 pc + rg
    const bool valid = t0 + kRowsPer * pc + rg < end;
    const float sc = valid ? score * scale : -INFINITY;
    const float nm = fmaxf(m, wave_max(sc));
    const float e = valid ? exp_nonpos_fast(sc - nm) : 0.0f;
    const float f = exp_nonpos_fast(m - nm);  // m = -inf on a wave's first tile: f = 0
    l = fmaf(l, f, wave_sum(e));
    m = nm;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc8[t] *= f;
    // the weight of row 8 j + rg is in lane 8 rg + j
    float ej[kPieces];
    ej[0] = group8_lane<0>(e);
    ej[1] = group8_lane<1>(e);
    ej[2] = group8_lane<2>(e);
    ej[3] = group8_lane<3>(e);
    ej[4] = group8_lane<4>(e);
    ej[5] = group8_lane<5>(e);
    ej[6] = group8_lane<6>(e);
    ej[7] = group8_lane<7>(e);
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
      // rows past the context hold whatever the cache held: never summed
      const bool row_ok = t0 + kRowsPer * j + rg < end;
      float vf[8];
      unpack8_bf16(vt[j], vf);
#pragma unroll
      for (int t = 0; t < 8; ++t) acc8[t] = row_ok ? fmaf(ej[j], vf[t], acc8[t]) : acc8[t];
      // one row's values unpacked at a time (registers)
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  tile(wave * kTile, kr, vr);
  if (kPrefetch) tile((wave + W) * kTile, kn, vn);
  const float mine = rows8_reduce_scatter(acc8, lane);  // dimension 8 pc + rg

  __shared__ float wm[W], wl[W];
  __shared__ float wacc[W][HD];
  if (lane == 0) {
    wm[wave] = m;
    wl[wave] = l;
  }
  wacc[wave][8 * pc + rg] = mine;
  __syncthreads();
  if (tid < HD) {
    float mm = wm[0];
#pragma unroll
    for (int w = 1; w < W; ++w) mm = fmaxf(mm, wm[w]);
    float ll = 0.0f, aa = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = wl[w] > 0.0f ? exp_nonpos_fast(wm[w] - mm) : 0.0f;
      ll = fmaf(wl[w], f, ll);
      aa = fmaf(wacc[w][tid], f, aa);
    }
    out[static_cast<size_t>(h) * HD + tid] = f32_to_bf16(aa / ll);
  }
}

// The whole-context attention in P parts (two halves, or four quarters):
// workgroup (query head h, part sp) takes the positions [sp * S, (sp + 1) *
// S) of the context, S = kAttnWholeMax / P, one 64-position tile per wave
// (S / 64 waves), all requested at kernel entry, and stores the part's
// (acc[HD], max, sum) record for the o-projection to merge
// (partial[(h * P + sp) * kAttnPartRecord]).  A part past the context exits
// without a record; the merge reads only parts [0, pos / S].  q is rotated
// and the caches hold the token's row (as the fused q|k|v launch leaves
// them).  Workgroups: part sp of kv head g on XCD (P g + sp) mod 8, each
// shared by the kv head's query heads (as whole_attention_head does for one
// workgroup per head).
int part_attention_blocks(int heads, int kv_heads, int parts) {
  const int units = parts * kv_heads;
  return kXcds * ((units + kXcds - 1) / kXcds) * (heads / kv_heads);
}

__device__ inline int part_attention_unit(int b, int heads, int kv_heads, int parts, int& h) {
  const int group = heads / kv_heads;
  const int x = b % kXcds, t = b / kXcds;
  const int u = (t / group) * kXcds + x;  // P g + sp
  h = (u / parts) * group + t % group;
  return u < parts * kv_heads ? u : -1;
}

template <int P>
__global__ __launch_bounds__(kAttnWholeMax / P / kTile * kWave) void attention_decode_parts_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ key_cache,
    const uint16_t* __restrict__ value_cache, const int* __restrict__ pos_ptr, int heads,
    int kv_heads, int max_seq, float* __restrict__ partial) {
  constexpr int HD = 64, S = kAttnWholeMax / P, W = S / kTile;
  constexpr int kPieces = HD / 8;            // 16-byte pieces per row (8)
  constexpr int kRowsPer = kWave / kPieces;  // rows per load instruction (8)
  static_assert(W * kTile == S, "one tile per wave covers a part");
  int h;
  const int u = part_attention_unit(blockIdx.x, heads, kv_heads, P, h);
  if (u < 0) return;
  const int g = u / P, sp = u % P;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int pc = lane % kPieces, rg = lane / kPieces;
  const size_t head_base = static_cast<size_t>(g) * max_seq * HD;
  const uint4 q_mine = reinterpret_cast<const uint4*>(q + static_cast<size_t>(h) * HD)[pc];
  // The tile goes out before the position arrives: rows past max_seq read 0,
  // rows past the context are masked below.
  const __amdgpu_buffer_rsrc_t kr_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(key_cache) + head_base, 0, max_seq * HD * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t vr_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(value_cache) + head_base, 0, max_seq * HD * 2, 0x00020000);
  const int t0 = sp * S + wave * kTile;
  uint4 kt[kPieces], vt[kPieces];
#pragma unroll
  for (int j = 0; j < kPieces; ++j) {
    const uint32_t off = static_cast<uint32_t>((t0 + kRowsPer * j + rg) * HD * 2 + 16 * pc);
    kt[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kr_rsrc, off, 0, 0));
  }
#pragma unroll
  for (int j = 0; j < kPieces; ++j) {
    const uint32_t off = static_cast<uint32_t>((t0 + kRowsPer * j + rg) * HD * 2 + 16 * pc);
    vt[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vr_rsrc, off, 0, 0));
  }
  const int end = min(*pos_ptr, max_seq - 1) + 1;  // positions [0, end)
  if (sp * S >= end) return;                       // a part past the context
  const float scale = 1.0f / sqrtf(static_cast<float>(HD));
  const uint32_t qw[4] = {q_mine.x, q_mine.y, q_mine.z, q_mine.w};
  float m = -INFINITY, l = 0.0f;
  float acc8[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc8[t] = 0.0f;
  if (t0 < end) {  // wave-uniform: a tile past the context is skipped whole
    float part[kPieces];
#pragma unroll
    for (int j = 0; j < kPieces; ++j) part[j] = dot8_packed_bf16(qw, kt[j]);
    const float score = group8_reduce_scatter(part, lane);  // row 8 pc + rg
    const bool valid = t0 + kRowsPer * pc + rg < end;
    const float sc = valid ? score * scale : -INFINITY;
    m = wave_max(sc);
    const float e = valid ? exp_nonpos_fast(sc - m) : 0.0f;
    l = wave_sum(e);
    float ej[kPieces];
    ej[0] = group8_lane<0>(e);
    ej[1] = group8_lane<1>(e);
    ej[2] = group8_lane<2>(e);
    ej[3] = group8_lane<3>(e);
    ej[4] = group8_lane<4>(e);
    ej[5] = group8_lane<5>(e);
    ej[6] = group8_lane<6>(e);
    ej[7] = group8_lane<7>(e);
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
      // rows past the context hold whatever the cache held: never summed
      const bool row_ok = t0 + kRowsPer * j + rg < end;
      float vf[8];
      unpack8_bf16(vt[j], vf);
#pragma unroll
      for (int t = 0; t < 8; ++t) acc8[t] = row_ok ? fmaf(ej[j], vf[t], acc8[t]) : acc8[t];
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  const float mine = rows8_reduce_scatter(acc8, lane);  // dimension 8 pc + rg
  __shared__ float wm[W], wl[W];
  __shared__ float wacc[W][HD];
  if (lane == 0) {
    wm[wave] = m;
    wl[wave] = l;
  }
  wacc[wave][8 * pc + rg] = mine;
  __syncthreads();
  if (tid < HD) {
    float mm = wm[0];
#pragma unroll
    for (int w = 1; w < W; ++w) mm = fmaxf(mm, wm[w]);
    float ll = 0.0f, aa = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = wl[w] > 0.0f ? exp_nonpos_fast(wm[w] - mm) : 0.0f;
      ll = fmaf(wl[w], f, ll);
      aa = fmaf(wacc[w][tid], f, aa);
    }
    float* rec = partial + static_cast<size_t>(h * P + sp) * kAttnPartRecord;
    rec[tid] = aa;
    if (tid == 0) {
      rec[HD] = mm;
      rec[HD + 1] = ll;
    }
  }
}

void launch_attention_decode_parts(const uint16_t* q, const uint16_t* key_cache,
                                   const uint16_t* value_cache, const int* pos, int heads,
                                   int kv_heads, int max_seq, float* partial,
                                   hipStream_t stream, int parts) {
  if (parts == 4) {
    hipLaunchKernelGGL(attention_decode_parts_kernel<4>,
                       dim3(part_attention_blocks(heads, kv_heads, 4)),
                       dim3(kAttnWholeMax / 4 / kTile * kWave), 0, stream, q, key_cache,
                       value_cache, pos, heads, kv_heads, max_seq, partial);
  } else {
    hipLaunchKernelGGL(attention_decode_parts_kernel<2>,
                       dim3(part_attention_blocks(heads, kv_heads, 2)),
                       dim3(kAttnWholeMax / 2 / kTile * kWave), 0, stream, q, key_cache,
                       value_cache, pos, heads, kv_heads, max_seq, partial);
  }
}

// ----------------------------------------------------- prefill attention --

// Causal attention of count tokens (positions 0 .. count - 1, already in
// the caches), the exact fallback for operands that are not 16-byte
// aligned: one wave per (query token, head), online softmax over the key
// positions 0 .. t in blocks of 64 (lane p scores key p of the block), then
// lane d accumulates output dimension d (and d + 64 when HD = 128).
template <int HD>
__global__ __launch_bounds__(kThreads) void attention_prefill_scalar_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ key_cache,
    const uint16_t* __restrict__ value_cache, uint16_t* __restrict__ out, int count, int heads,
    int kv_heads, int max_seq) {
  constexpr int kDims = HD / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int item = blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
  if (item >= count * heads) return;
  const int t = item / heads, h = item % heads;
  const int g = h / (heads / kv_heads);
  __shared__ float wts[kThreads / kWave][kWave];
  float* wt = wts[threadIdx.x / kWave];
  const uint16_t* qh = q + (static_cast<size_t>(t) * heads + h) * HD;
  float qv[HD];
#pragma unroll
  for (int d = 0; d < HD; ++d) qv[d] = load_bf16(qh + d);
  const float scale = 1.0f / sqrtf(static_cast<float>(HD));
  const uint16_t* kbase = key_cache + static_cast<size_t>(g) * max_seq * HD;
  const uint16_t* vbase = value_cache + static_cast<size_t>(g) * max_seq * HD;
  float m = -INFINITY, l = 0.0f;
  float acc[kDims];
#pragma unroll
  for (int j = 0; j < kDims; ++j) acc[j] = 0.0f;
  for (int p0 = 0; p0 <= t; p0 += kWave) {
    const int p = p0 + lane;
    float s = -INFINITY;
    if (p <= t) {
      // 2-byte loads: this kernel serves operands of any (2-byte) alignment
      const uint16_t* kr = kbase + static_cast<size_t>(p) * HD;
      float dot = 0.0f;
#pragma unroll
      for (int d = 0; d < HD; ++d) dot = fmaf(qv[d], load_bf16(kr + d), dot);
      s = dot * scale;
    }
    const float bm = wave_max(s);
    const float nm = fmaxf(m, bm);
    const float e = p <= t ? expf(s - nm) : 0.0f;
    const float f = expf(m - nm);  // m = -inf on the first block: f = 0
    l = fmaf(l, f, wave_sum(e));
#pragma unroll
    for (int j = 0; j < kDims; ++j) acc[j] *= f;
    wt[lane] = e;
    __builtin_amdgcn_wave_barrier();
    const int n = min(kWave, t - p0 + 1);
#pragma unroll 8
    for (int pp = 0; pp < n; ++pp) {
      const uint16_t* vr = vbase + static_cast<size_t>(p0 + pp) * HD + lane;
#pragma unroll
      for (int j = 0; j < kDims; ++j) acc[j] = fmaf(wt[pp], load_bf16(vr + kWave * j), acc[j]);
    }
    __builtin_amdgcn_wave_barrier();
    m = nm;
  }
#pragma unroll
  for (int j = 0; j < kDims; ++j) {
    out[(static_cast<size_t>(t) * heads + h) * HD + lane + kWave * j] = f32_to_bf16(acc[j] / l);
  }
}

// Causal prefill attention on MFMA (v_mfma_f32_32x32x16_bf16).  Workgroup
// (query block b, head h) takes the 32 queries 32 b .. 32 b + 31; its W
// waves take the 32-key blocks 0 .. b round robin (block w, w + W, ...), each
// with its own online softmax, and are merged in LDS at the end.
//
// Per key block a wave computes S^T = K Q^T (keys x queries) rather than
// S = Q K^T: in the accumulator layout lane (r, h) = (lane % 32, lane / 32)
// then holds query r and the 16 keys 8 (e / 4) + 4 h + e % 4 (e < 16), so a
// query's max and sum are 16 in-register values plus one exchange with lane
// r + 32.  The probabilities are already laid out as the B operand of
// O^T = V^T P^T (k-step s takes accumulator elements 8 s .. 8 s + 7, i.e. keys
// 16 s + 4 h + 0..3 and 16 s + 8 + 4 h + 0..3), and O^T's column is the
// lane's own query, so the online-softmax rescale needs no exchange at all.
// V^T's A fragments need the same key order per dimension: the block's value
// rows go through the wave's LDS slice transposed (4 keys packed per
// 8-byte write), and each fragment is then two 8-byte reads.  P is split
// into BF16 hi + lo parts (two MFMAs each), so P V keeps about 16 bits of
// each probability instead of 8: the result stays within a few FP32 ulps of
// the reference's FP32 loop rather than BF16 rounding of P.  The
// exponentials are the hardware's 2^x (v_exp_f32) on scores pre-scaled by
// scale * log2(e), one FMA and one transcendental per score instead of
// expf's range reduction: the loop is VALU-bound, and this cut a 512-token
// launch from 8.7 to 6.3 us (errors stay well under the output's BF16
// rounding).
typedef __bf16 attn_bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 attn_bf16x4_t __attribute__((ext_vector_type(4)));
typedef float attn_f32x16_t __attribute__((ext_vector_type(16)));
typedef float attn_f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 attn_bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kPrefillQueries = 32;     // queries per workgroup
constexpr int kPrefillVtStride = 36;    // BF16 words per transposed value row (32 keys + pad)
constexpr float kPrefillLazyLog2 = 8.0f;  // the softmax reference's slack (log2 units)
#ifndef QLIN_PREFILL_WAVES64
#define QLIN_PREFILL_WAVES64 4
#endif
// Waves per workgroup at head_dim 64 (head_dim 128: 4).  Measured on the
// 512-token prefill of Qwen2.5-0.5B (16 x 14 workgroups): 5.72 us per launch
// with 4 waves, 6.69 with 8 (6.32 against 7.04 with expf and a rescale every
// block): two waves per SIMD add no throughput to a loop that is VALU-bound,
// and the 8-way merge costs more.
constexpr int kPrefillWaves64 = QLIN_PREFILL_WAVES64;

template <int HD, int W>
struct alignas(16) PrefillSmem {
  // per wave: V^T of one key block while its blocks run, then its O^T
  union alignas(16) Slice {
    uint16_t vt[HD * kPrefillVtStride];
    float o[HD][kPrefillQueries + 1];
  } w[W];
  float m[W][kPrefillQueries];
  float l[W][kPrefillQueries];
};

__device__ __forceinline__ float swap32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false,
                                                  false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}

// ROPE: q, k and v come unrotated from the q|k|v GEMM (k and v [count]
// [kv_heads][HD]): q is rotated as it is loaded, each key block as it
// arrives (rope_store_rows_kernel's arithmetic on the same BF16 values,
// rounded to BF16), and the workgroup of each kv head's first query head
// stores its diagonal key block, rotated, and the block's values into the
// caches.  The prefill's own RoPE + KV store launch then does not run.
struct PrefillRope {
  const uint16_t* k = nullptr;
  const uint16_t* v = nullptr;
  const float2* table = nullptr;  // [max_seq][HD / 2] (cos, sin)
};

// (a, b) = (a cos - b sin, b cos + a sin) on each BF16 pair of (lo, hi),
// rounded to BF16 (rope_store_rows_kernel's arithmetic).
__device__ __forceinline__ void rope_bf16x8(uint4& lo, uint4& hi, const float2 (&cs)[8]) {
  const uint32_t l4[4] = {lo.x, lo.y, lo.z, lo.w}, h4[4] = {hi.x, hi.y, hi.z, hi.w};
  uint32_t ol[4], oh[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float a0 = bf16_lo(l4[e]), b0 = bf16_lo(h4[e]);
    float a1 = bf16_hi(l4[e]), b1 = bf16_hi(h4[e]);
    rope_pair(a0, b0, cs[2 * e]);
    rope_pair(a1, b1, cs[2 * e + 1]);
    ol[e] = pack2_bf16(a0, a1);
    oh[e] = pack2_bf16(b0, b1);
  }
  lo = make_uint4(ol[0], ol[1], ol[2], ol[3]);
  hi = make_uint4(oh[0], oh[1], oh[2], oh[3]);
}

template <int HD, int W, bool ROPE>
__global__ __launch_bounds__(W * kWave) void attention_prefill_mfma_kernel(
    const uint16_t* __restrict__ q, uint16_t* __restrict__ key_cache,
    uint16_t* __restrict__ value_cache, uint16_t* __restrict__ out, int count, int heads,
    int kv_heads, int max_seq, PrefillRope pr) {
  constexpr int KS = HD / 16;          // k-steps of S^T (16 dimensions each)
  constexpr int DT = HD / 32;          // 32-dimension row tiles of O^T
  constexpr int kChunks = HD / 8;      // 16-byte chunks per row
  constexpr int VC = 8 * kChunks / 64; // (key quad, chunk) pairs per lane
  __shared__ PrefillSmem<HD, W> sm;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 31, h = lane >> 5;
  const int qb = blockIdx.x, head = blockIdx.y;
  const int g = head / (heads / kv_heads);
  const int q0 = qb * kPrefillQueries;
  const int query = q0 + r;
  const float scale = 1.0f / sqrtf(static_cast<float>(HD));
  const float scale_log2 = scale * 1.44269504088896340736f;  // scale * log2(e)

  // Q^T fragments (B of S^T): lane (r, h) holds dimensions 16 ks + 8 h .. + 7
  // of query r (rows past count are clamped; their results are dropped).
  attn_bf16x8_t qf[KS];
  {
    const uint16_t* qp =
        q + (static_cast<size_t>(min(query, count - 1)) * heads + head) * HD + 8 * h;
    uint4 qr[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qr[ks] = load_global16(qp + 16 * ks);
    if (ROPE) {  // pairs (i, i + HD / 2): chunks ks and ks + KS / 2 of this lane
      const float2* cs = pr.table + static_cast<size_t>(min(query, count - 1)) * (HD / 2) + 8 * h;
#pragma unroll
      for (int ks = 0; ks < KS / 2; ++ks) {
        float2 c8[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) c8[j] = cs[16 * ks + j];
        rope_bf16x8(qr[ks], qr[ks + KS / 2], c8);
      }
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = __builtin_bit_cast(attn_bf16x8_t, qr[ks]);
  }
  // The kv head's cache rows as buffer resources: a block's loads are a
  // scalar offset (its first key) over per-lane offsets fixed for the whole
  // loop, and rows at or past max_seq read as zero.
  // (ROPE: the q|k|v GEMM's k and v rows of the kv head, kv_heads * HD
  // apart; rows at or past count read as zero.)
  const int kv_row = ROPE ? kv_heads * HD : HD;  // elements between key rows
  const uint32_t head_bytes =
      ROPE ? static_cast<uint32_t>((count - 1) * kv_row + HD) * 2
           : static_cast<uint32_t>(max_seq) * HD * 2;
  const uint16_t* ksrc =
      ROPE ? pr.k + static_cast<size_t>(g) * HD : key_cache + static_cast<size_t>(g) * max_seq * HD;
  const uint16_t* vsrc = ROPE ? pr.v + static_cast<size_t>(g) * HD
                              : value_cache + static_cast<size_t>(g) * max_seq * HD;
  const __amdgpu_buffer_rsrc_t kres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(ksrc), 0, static_cast<int>(head_bytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t vres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(vsrc), 0, static_cast<int>(head_bytes), 0x00020000);
  uint16_t* vt = sm.w[wave].vt;

  float m = -INFINITY, l = 0.0f;
  attn_f32x16_t o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.0f;

  // Loads of key block kb: K rows (A of S^T, lane (r, h): key r, dimensions
  // 16 ks + 8 h ..) and the value chunks this lane transposes (pair i:
  // keys 4 a .. 4 a + 3, dimensions 8 c .. 8 c + 7).  Keys past max_seq
  // read as zero; keys past count are masked (K) or zeroed (V).
  const uint32_t koff = static_cast<uint32_t>(r * kv_row + 8 * h) * 2;
  uint32_t voff[VC];
#pragma unroll
  for (int i = 0; i < VC; ++i) {
    const int idx = lane + 64 * i;
    voff[i] = static_cast<uint32_t>(4 * (idx / kChunks) * kv_row + 8 * (idx % kChunks)) * 2;
  }
  uint4 kr[KS], vr[VC][4];
  float2 kcs[ROPE ? KS / 2 : 1][8];  // ROPE: (cos, sin) of key row r's pairs
  auto load_block = [&](int kb) {
    const int k0 = kb * 32;
    const uint32_t soff = static_cast<uint32_t>(k0) * kv_row * 2;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      kr[ks] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(kres, koff + 32 * ks, soff, 0));
    }
#pragma unroll
    for (int i = 0; i < VC; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        vr[i][j] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(vres, voff[i] + j * kv_row * 2, soff, 0));
      }
    if (ROPE) {
      const float2* cs =
          pr.table + static_cast<size_t>(min(k0 + r, count - 1)) * (HD / 2) + 8 * h;
#pragma unroll
      for (int ks = 0; ks < KS / 2; ++ks)
#pragma unroll
        for (int j = 0; j < 8; ++j) kcs[ks][j] = cs[16 * ks + j];
    }
    if (k0 + 32 > count) {  // only the last block reaches past count
#pragma unroll
      for (int i = 0; i < VC; ++i) {
        const int a = (lane + 64 * i) / kChunks;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (k0 + 4 * a + j >= count) vr[i][j] = make_uint4(0, 0, 0, 0);
      }
    }
  };

  int kb = wave;
  if (kb <= qb) load_block(kb);
  for (; kb <= qb; kb += W) {
    const int k0 = kb * 32;
    if (ROPE) {
#pragma unroll
      for (int ks = 0; ks < KS / 2; ++ks) rope_bf16x8(kr[ks], kr[ks + KS / 2], kcs[ks]);
      if (kb == qb && head % (heads / kv_heads) == 0) {
        // the diagonal block into the caches: rotated key rows, value rows
        uint16_t* kc = key_cache + static_cast<size_t>(g) * max_seq * HD;
        uint16_t* vc = value_cache + static_cast<size_t>(g) * max_seq * HD;
        const int key = k0 + r;
        if (key < count && key < max_seq) {
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            store_global16(kc + static_cast<size_t>(key) * HD + 16 * ks + 8 * h, kr[ks]);
          }
        }
#pragma unroll
        for (int i = 0; i < VC; ++i) {
          const int idx = lane + 64 * i, a = idx / kChunks, c = idx % kChunks;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int vkey = k0 + 4 * a + j;
            if (vkey < count && vkey < max_seq) {
              store_global16(vc + static_cast<size_t>(vkey) * HD + 8 * c, vr[i][j]);
            }
          }
        }
      }
    }
    // transpose this block's values into vt[d][key]: 4 keys per 8-byte write
    __builtin_amdgcn_wave_barrier();  // the previous block's reads are done
#pragma unroll
    for (int i = 0; i < VC; ++i) {
      const int idx = lane + 64 * i, a = idx / kChunks, c = idx % kChunks;
      const uint32_t w[4][4] = {{vr[i][0].x, vr[i][0].y, vr[i][0].z, vr[i][0].w},
                                {vr[i][1].x, vr[i][1].y, vr[i][1].z, vr[i][1].w},
                                {vr[i][2].x, vr[i][2].y, vr[i][2].z, vr[i][2].w},
                                {vr[i][3].x, vr[i][3].y, vr[i][3].z, vr[i][3].w}};
#pragma unroll
      for (int p = 0; p < 4; ++p) {  // dimensions 8 c + 2 p, 8 c + 2 p + 1
        // selector 0x05040100: low halves of (src1, src0); 0x07060302: high halves
        const uint32_t lo01 = __builtin_amdgcn_perm(w[1][p], w[0][p], 0x05040100u);
        const uint32_t lo23 = __builtin_amdgcn_perm(w[3][p], w[2][p], 0x05040100u);
        const uint32_t hi01 = __builtin_amdgcn_perm(w[1][p], w[0][p], 0x07060302u);
        const uint32_t hi23 = __builtin_amdgcn_perm(w[3][p], w[2][p], 0x07060302u);
        *reinterpret_cast<uint2*>(vt + (8 * c + 2 * p) * kPrefillVtStride + 4 * a) =
            make_uint2(lo01, lo23);
        *reinterpret_cast<uint2*>(vt + (8 * c + 2 * p + 1) * kPrefillVtStride + 4 * a) =
            make_uint2(hi01, hi23);
      }
    }
    // S^T = K Q^T
    attn_f32x16_t st;
#pragma unroll
    for (int e = 0; e < 16; ++e) st[e] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(attn_bf16x8_t, kr[ks]),
                                                   qf[ks], st, 0, 0, 0);
    }
    if (kb + W <= qb) load_block(kb + W);  // next block in flight
    // causal mask (only the diagonal block holds keys past a query), online
    // softmax of query r over this block in base 2 with x = s * scale *
    // log2(e): p = 2^(x - m) for a reference m that moves (rescaling l and
    // the accumulators by 2^(m_old - m_new)) only when a score of the wave's
    // queries exceeds it by more than kPrefillLazyLog2, so p <= 2^8 and most
    // blocks skip the rescale.  The final division by l removes m exactly;
    // the BF16 hi + lo split keeps the same relative precision of p at any
    // scale.  (max(s) * c = max(s * c) for c > 0, rounding being monotonic.)
    if (kb == qb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = k0 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (key > query) st[e] = -INFINITY;
      }
    }
    float bm = st[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) bm = fmaxf(bm, st[e]);
    bm = swap32_max(bm) * scale_log2;
    // m = -inf before the first block: every wave rescales there (f = 0)
    if (__builtin_amdgcn_ballot_w64(bm > m + kPrefillLazyLog2) != 0) {
      const float mn = fmaxf(m, bm);
      const float f = __builtin_amdgcn_exp2f(m - mn);
      l *= f;
      m = mn;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] *= f;
    }
    float ps = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      st[e] = __builtin_amdgcn_exp2f(fmaf(st[e], scale_log2, -m));
      ps += st[e];
    }
    l += swap32_sum(ps, ps);
    __builtin_amdgcn_wave_barrier();  // vt complete for the whole wave
    // O^T += V^T (P_hi + P_lo)^T
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      attn_bf16x8_t phi, plo;
#pragma unroll
      for (int j = 0; j < 4; ++j) {  // two probabilities per conversion
        const attn_f32x2_t p = {st[8 * s + 2 * j], st[8 * s + 2 * j + 1]};
        const attn_bf16x2_t hi = __builtin_convertvector(p, attn_bf16x2_t);
        const attn_bf16x2_t lo =
            __builtin_convertvector(p - __builtin_convertvector(hi, attn_f32x2_t), attn_bf16x2_t);
        phi[2 * j] = hi[0];
        phi[2 * j + 1] = hi[1];
        plo[2 * j] = lo[0];
        plo[2 * j + 1] = lo[1];
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint16_t* vrow = vt + (32 * dt + r) * kPrefillVtStride + 16 * s + 4 * h;
        const uint2 v0 = *reinterpret_cast<const uint2*>(vrow);
        const uint2 v1 = *reinterpret_cast<const uint2*>(vrow + 8);
        const attn_bf16x8_t va =
            __builtin_bit_cast(attn_bf16x8_t, make_uint4(v0.x, v0.y, v1.x, v1.y));
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, phi, o[dt], 0, 0, 0);
        o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, plo, o[dt], 0, 0, 0);
      }
    }
  }

  // merge the waves: O^T element e of tile dt is dimension 32 dt + 8 (e / 4)
  // + 4 h + e % 4 of query r.  O^T overwrites the wave's V^T slice: the
  // compiler barrier keeps these stores after the last block's V^T reads
  // (float and BF16 accesses are otherwise taken as disjoint), and the wave's
  // LDS operations execute in order.
  asm volatile("" ::: "memory");
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) sm.w[wave].o[32 * dt + 8 * (e >> 2) + 4 * h + (e & 3)][r] = o[dt][e];
  if (h == 0) {
    sm.m[wave][r] = m;
    sm.l[wave][r] = l;
  }
  __syncthreads();
  constexpr int kItems = kPrefillQueries * kChunks;  // (query, 8-dimension chunk)
#pragma unroll
  for (int it = threadIdx.x; it < kItems; it += W * kWave) {
    const int qi = it / kChunks, c = it % kChunks;
    if (q0 + qi >= count) continue;
    float mm = sm.m[0][qi];
#pragma unroll
    for (int w = 1; w < W; ++w) mm = fmaxf(mm, sm.m[w][qi]);
    float cw[W], den = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      cw[w] = __builtin_amdgcn_exp2f(sm.m[w][qi] - mm);  // a wave with no block: m = -inf, weight 0
      den = fmaf(sm.l[w][qi], cw[w], den);
    }
    const float inv = 1.0f / den;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float a = 0.0f;
#pragma unroll
      for (int w = 0; w < W; ++w) a = fmaf(sm.w[w].o[8 * c + j][qi], cw[w], a);
      acc[j] = a * inv;
    }
    uint16_t* dst = out + (static_cast<size_t>(q0 + qi) * heads + head) * HD + 8 * c;
    *reinterpret_cast<uint4*>(dst) =
        make_uint4(pack2_bf16(acc[0], acc[1]), pack2_bf16(acc[2], acc[3]),
                   pack2_bf16(acc[4], acc[5]), pack2_bf16(acc[6], acc[7]));
  }
}

// -------------------------------------------------------- elementwise --

__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const uint16_t* __restrict__ gate,
                                                            const uint16_t* __restrict__ up,
                                                            uint16_t* __restrict__ out,
                                                            long long n) {
  for (long long i = blockIdx.x * static_cast<long long>(kThreads) + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * kThreads) {
    const float g = load_bf16(gate + i);
    out[i] = f32_to_bf16(g / (1.0f + expf(-g)) * load_bf16(up + i));
  }
}

__global__ __launch_bounds__(kThreads) void add_kernel(uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ y,
                                                       long long n) {
  for (long long i = blockIdx.x * static_cast<long long>(kThreads) + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * kThreads) {
    x[i] = f32_to_bf16(load_bf16(x + i) + load_bf16(y + i));
  }
}

// Host-chosen decode state (a kernel, not a copy, so that it can sit in a
// captured graph).  token < 0 keeps the current token.
__global__ void set_state_kernel(ModelState* state, int token, int pos, int step,
                                 RopeCursor rope, unsigned long long* key) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    if (token >= 0) state->token = token;
    state->pos = pos;
    state->step = step;
    if (key) __hip_atomic_store(key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (rope.row && static_cast<int>(threadIdx.x) < rope.half) {
    rope.row[threadIdx.x] =
        rope.table[static_cast<size_t>(min(pos, rope.max_seq - 1)) * rope.half + threadIdx.x];
  }
}
__global__ void advance_kernel(ModelState* state, int* __restrict__ history, int history_len,
                               RopeCursor rope) {
  const int pos = state->pos;
  if (rope.row && static_cast<int>(threadIdx.x) < rope.half) {
    rope.row[threadIdx.x] =
        rope.table[static_cast<size_t>(min(pos + 1, rope.max_seq - 1)) * rope.half +
                   threadIdx.x];
  }
  __syncthreads();  // every lane has read pos before thread 0 moves it on
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    const int step = state->step;
    if (step < history_len) history[step] = state->token;
    state->step = step + 1;
    state->pos = pos + 1;
  }
}

// ------------------------------------------------------------ launchers --

namespace {
int grid_for(long long n) {
  const long long b = (n + kThreads - 1) / kThreads;
  return static_cast<int>(b < 4096 ? (b > 0 ? b : 1) : 4096);
}
}  // namespace

void launch_embedding(const uint16_t* table, const int* tokens, int count, int vocab, int hidden,
                      uint16_t* out, hipStream_t stream) {
  hipLaunchKernelGGL(embedding_kernel, dim3(count), dim3(kThreads), 0, stream, table, tokens,
                     count, vocab, hidden, out);
}

void launch_embedding_rms_norm(const uint16_t* table, const int* tokens, int count, int vocab,
                               int hidden, uint16_t* x, const uint16_t* w, uint16_t* out,
                               float eps, hipStream_t stream) {
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  const int ch = a16(table) ? norm_rows_chunks(x, nullptr, w, out, hidden) : 0;
  if (ch) {
    launch_norm_rows<false, true>(ch, x, nullptr, w, out, count, hidden, eps, stream, table,
                                  tokens, vocab);
    return;
  }
  launch_embedding(table, tokens, count, vocab, hidden, x, stream);
  launch_rms_norm(x, w, out, count, hidden, eps, stream);
}

void launch_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* out, int rows, int hidden,
                     float eps, hipStream_t stream) {
  if (const int ch = norm_rows_chunks(x, nullptr, w, out, hidden)) {
    launch_norm_rows<false>(ch, const_cast<uint16_t*>(x), nullptr, w, out, rows, hidden, eps,
                            stream);
    return;
  }
  hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(kThreads), 0, stream, x, w, out, rows,
                     hidden, eps);
}

void launch_add_rms_norm(uint16_t* x, const uint16_t* y, const uint16_t* w, uint16_t* out,
                         int rows, int hidden, float eps, hipStream_t stream) {
  if (const int ch = norm_rows_chunks(x, y, w, out, hidden)) {
    launch_norm_rows<true>(ch, x, y, w, out, rows, hidden, eps, stream);
    return;
  }
  hipLaunchKernelGGL(add_rms_norm_kernel, dim3(rows), dim3(kThreads), 0, stream, x, y, w, out,
                     rows, hidden, eps);
}

void launch_rope_store(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* key_cache,
                       uint16_t* value_cache, const float2* rope, int count, int start,
                       int heads, int kv_heads, int head_dim, int max_seq,
                       hipStream_t stream) {
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (head_dim % 16 == 0 && a16(q) && a16(k) && a16(v) && a16(key_cache) &&
      a16(value_cache) && a16(rope)) {
    hipLaunchKernelGGL(rope_store_rows_kernel,
                       dim3((count + kThreads / kWave - 1) / (kThreads / kWave)), dim3(kThreads),
                       0, stream, q, k, v, key_cache, value_cache, rope, count, start, heads,
                       kv_heads, head_dim, max_seq);
    return;
  }
  hipLaunchKernelGGL(rope_store_kernel, dim3(count), dim3(kThreads), 0, stream, q, k, v,
                     key_cache, value_cache, rope, count, start, heads, kv_heads, head_dim,
                     max_seq);
}

bool attention_head_dim_supported(int head_dim) { return head_dim == 64 || head_dim == 128; }

bool attention_whole(int max_seq, int head_dim) {
  return head_dim == 64 && max_seq <= kAttnWholeMax;
}

int attention_span(int max_seq, int head_dim) {
  if (attention_whole(max_seq, head_dim)) return kAttnWholeMax;
  // Spans of kAttnWaves 64-position tiles (one tile per wave), widened so
  // that a context has at most kAttnMaxSplits spans.
  const int base = kAttnWaves * kTile;
  const int need = (max_seq + kAttnMaxSplits - 1) / kAttnMaxSplits;
  const int tiles = (need + base - 1) / base;
  return base * (tiles > 1 ? tiles : 1);
}

int attention_splits(int max_seq, int head_dim) {
  const int span = attention_span(max_seq, head_dim);
  return (max_seq + span - 1) / span;
}

void launch_attention_decode(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                             uint16_t* key_cache, uint16_t* value_cache, const float2* rope,
                             const int* pos, int heads, int kv_heads, int head_dim,
                             int max_seq, bool roped, float* partial, uint16_t* out,
                             hipStream_t stream) {
  if (attention_whole(max_seq, head_dim) && roped) {
    hipLaunchKernelGGL(attention_decode_whole_kernel,
                       dim3(whole_attention_blocks(heads, kv_heads)), dim3(kWholeWaves * kWave),
                       0, stream, q, key_cache, value_cache, pos, heads, kv_heads, max_seq, out);
    return;
  }
  const int span = attention_span(max_seq, head_dim);
  const int splits = attention_splits(max_seq, head_dim);
  const dim3 grid(splits, heads), block(kAttnWaves * kWave);
#define QLIN_SPANS(HDV, R)                                                                      \
  hipLaunchKernelGGL((attention_decode_kernel<HDV, R>), grid, block, 0, stream, q, k_new, v_new, \
                     key_cache, value_cache, rope, pos, heads, kv_heads, max_seq, span, splits,  \
                     partial)
  if (head_dim == 64) {
    if (roped) {
      QLIN_SPANS(64, true);
    } else {
      QLIN_SPANS(64, false);
    }
  } else {
    if (roped) {
      QLIN_SPANS(128, true);
    } else {
      QLIN_SPANS(128, false);
    }
  }
#undef QLIN_SPANS
}

void launch_attention_decode_spans(const uint16_t* q, const uint16_t* key_cache,
                                   const uint16_t* value_cache, const int* pos, int heads,
                                   int kv_heads, int head_dim, int max_seq, float* partial,
                                   hipStream_t stream) {
  // the split form even where the whole-context one applies (span
  // kAttnWholeMax, one split), pre-rotated
  const int span = attention_span(max_seq, head_dim);
  const int splits = attention_splits(max_seq, head_dim);
  const dim3 grid(splits, heads), block(kAttnWaves * kWave);
  uint16_t* kc = const_cast<uint16_t*>(key_cache);
  uint16_t* vc = const_cast<uint16_t*>(value_cache);
  if (head_dim == 64) {
    hipLaunchKernelGGL((attention_decode_kernel<64, true>), grid, block, 0, stream, q, nullptr,
                       nullptr, kc, vc, nullptr, pos, heads, kv_heads, max_seq, span, splits,
                       partial);
  } else {
    hipLaunchKernelGGL((attention_decode_kernel<128, true>), grid, block, 0, stream, q, nullptr,
                       nullptr, kc, vc, nullptr, pos, heads, kv_heads, max_seq, span, splits,
                       partial);
  }
}

bool attention_prefill_rope(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            uint16_t* key_cache, uint16_t* value_cache, const float2* rope,
                            uint16_t* out, int count, int heads, int kv_heads, int head_dim,
                            int max_seq, hipStream_t stream) {
  const bool aligned =
      ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
        reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(key_cache) |
        reinterpret_cast<uintptr_t>(value_cache) | reinterpret_cast<uintptr_t>(rope) |
        reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
  if (!aligned || count < 1 || count > kPrefillRopeMaxTokens || count > max_seq ||
      (head_dim != 64 && head_dim != 128)) {
    return false;
  }
  const dim3 grid((count + kPrefillQueries - 1) / kPrefillQueries, heads);
  const PrefillRope pr{k, v, rope};
  if (head_dim == 64) {
    hipLaunchKernelGGL((attention_prefill_mfma_kernel<64, kPrefillWaves64, true>), grid,
                       dim3(kPrefillWaves64 * kWave), 0, stream, q, key_cache, value_cache, out,
                       count, heads, kv_heads, max_seq, pr);
  } else {
    hipLaunchKernelGGL((attention_prefill_mfma_kernel<128, 4, true>), grid, dim3(4 * kWave), 0,
                       stream, q, key_cache, value_cache, out, count, heads, kv_heads, max_seq,
                       pr);
  }
  return true;
}

void launch_attention_prefill(const uint16_t* q, const uint16_t* key_cache,
                              const uint16_t* value_cache, uint16_t* out, int count, int heads,
                              int kv_heads, int head_dim, int max_seq, hipStream_t stream) {
  const bool aligned = ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(key_cache) |
                         reinterpret_cast<uintptr_t>(value_cache) |
                         reinterpret_cast<uintptr_t>(out)) & 15u) == 0;
  // The MFMA kernel addresses a kv head's cache rows through a buffer
  // resource (32-bit byte offsets).
  const bool offsets32 =
      static_cast<long long>(max_seq) * head_dim * 2 <= static_cast<long long>(INT32_MAX);
  if (aligned && offsets32) {
    const dim3 grid((count + kPrefillQueries - 1) / kPrefillQueries, heads);
    uint16_t* kc = const_cast<uint16_t*>(key_cache);
    uint16_t* vc = const_cast<uint16_t*>(value_cache);
    if (head_dim == 64) {
      hipLaunchKernelGGL((attention_prefill_mfma_kernel<64, kPrefillWaves64, false>), grid,
                         dim3(kPrefillWaves64 * kWave), 0, stream, q, kc, vc, out, count, heads,
                         kv_heads, max_seq, PrefillRope{});
    } else {
      hipLaunchKernelGGL((attention_prefill_mfma_kernel<128, 4, false>), grid, dim3(4 * kWave),
                         0, stream, q, kc, vc, out, count, heads, kv_heads, max_seq,
                         PrefillRope{});
    }
    return;
  }
  const int waves = count * heads;
  const int blocks = (waves + kThreads / kWave - 1) / (kThreads / kWave);
  if (head_dim == 64) {
    hipLaunchKernelGGL(attention_prefill_scalar_kernel<64>, dim3(blocks), dim3(kThreads), 0,
                       stream, q, key_cache, value_cache, out, count, heads, kv_heads, max_seq);
  } else {
    hipLaunchKernelGGL(attention_prefill_scalar_kernel<128>, dim3(blocks), dim3(kThreads), 0,
                       stream, q, key_cache, value_cache, out, count, heads, kv_heads, max_seq);
  }
}

void launch_silu_mul(const uint16_t* gate, const uint16_t* up, uint16_t* out, long long n,
                     hipStream_t stream) {
  hipLaunchKernelGGL(silu_mul_kernel, dim3(grid_for(n)), dim3(kThreads), 0, stream, gate, up, out,
                     n);
}

void launch_add(uint16_t* x, const uint16_t* y, long long n, hipStream_t stream) {
  hipLaunchKernelGGL(add_kernel, dim3(grid_for(n)), dim3(kThreads), 0, stream, x, y, n);
}

void launch_set_state(ModelState* state, int token, int pos, int step, RopeCursor rope,
                      hipStream_t stream, unsigned long long* key) {
  hipLaunchKernelGGL(set_state_kernel, dim3(1), dim3(kWave * 2), 0, stream, state, token, pos,
                     step, rope, key);
}

__global__ __launch_bounds__(kThreads) void decode_entry_kernel(DecodeEntryArgs a) {
  __shared__ int s_token, s_pos;
  if (threadIdx.x == 0) {
    // the key and the state in one round trip
    const unsigned long long key =
        __hip_atomic_load(a.key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ModelState* st = a.state;
    int token = st->token, pos = st->pos;
    const int step = st->step;
    if (key >> 63) {
      token = lm_key_row(key);
      if (step < a.history_len) a.history[step] = token;
      st->step = step + 1;
      st->token = token;
      st->pos = ++pos;
      __hip_atomic_store(a.key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    s_token = token;
    s_pos = pos;
  }
  __syncthreads();
  if (a.rope.row && static_cast<int>(threadIdx.x) < a.rope.half) {
    a.rope.row[threadIdx.x] =
        a.rope.table[static_cast<size_t>(min(s_pos, a.rope.max_seq - 1)) * a.rope.half +
                     threadIdx.x];
  }
  if (!a.out) return;
  const int token = min(max(s_token, 0), a.vocab - 1);
  const uint16_t* src = a.table + static_cast<size_t>(token) * a.hidden;
  if ((a.hidden & 7) == 0) {
    for (int c = threadIdx.x; c < a.hidden / 8; c += kThreads) {
      reinterpret_cast<uint4*>(a.out)[c] = reinterpret_cast<const uint4*>(src)[c];
    }
  } else {
    for (int c = threadIdx.x; c < a.hidden; c += kThreads) a.out[c] = src[c];
  }
}

void launch_decode_entry(const DecodeEntryArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(decode_entry_kernel, dim3(1), dim3(kThreads), 0, stream, a);
}

void launch_advance(ModelState* state, int* history, int history_len, RopeCursor rope,
                    hipStream_t stream) {
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(kWave * 2), 0, stream, state, history,
                     history_len, rope);
}

}  // namespace qlin
