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

// ------------------------------------------------------- RoPE + KV store --

// Rotate one head (head_dim values, pairs (i, i + half)) by the angles of
// `position`; `rope` holds (cos, sin) for [position][i].
__device__ __forceinline__ void rope_pair(float& a, float& b, float2 cs) {
  const float first = a, second = b;
  a = first * cs.x - second * cs.y;
  b = second * cs.x + first * cs.y;
}

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

// ------------------------------------------------------ decode attention --

// One decode step's attention for every head, split over the context.
// Workgroup (c, g) takes positions [c * kChunk, (c + 1) * kChunk) of the
// context [0, pos] for the `group` query heads of kv head g.  Every
// workgroup rotates the group's q in LDS; the chunk holding pos also
// rotates that token's k and stores its k and v into the caches (no other
// workgroup reads position pos: the chunk's own reads of that row take the
// new values from k_new / v_new).  The chunk's value rows are staged in LDS
// with 16-byte loads; lane p scores position p (its key row as 16-byte
// loads), lane d accumulates output dimension d (and d + 64 when HD = 128).
// Each workgroup writes its per-head (acc[HD], max, sum) partial; the last
// one of kv head g to finish (counted on counters[g] with device-coherent
// accesses) merges the partials in chunk order, writes the heads' BF16
// outputs and resets its counter.  A context of one chunk skips the merge.
constexpr int kChunk = 64;

template <int HD>
__global__ __launch_bounds__(kThreads) void attention_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_new,
    const uint16_t* __restrict__ v_new, uint16_t* __restrict__ key_cache,
    uint16_t* __restrict__ value_cache, const float2* __restrict__ rope,
    const ModelState* __restrict__ state, int heads, int kv_heads, int max_seq,
    float* __restrict__ partial, int* __restrict__ counters, uint16_t* __restrict__ out) {
  constexpr int half = HD / 2;
  constexpr int kDims = HD / kWave;     // output dimensions per lane
  constexpr int kPieces = HD / 8;       // 16-byte pieces per cache row
  constexpr int kWaves = kThreads / kWave;
  constexpr int kRec = HD + 2;          // partial record: acc[HD], max, sum
  const int g = blockIdx.y;
  const int c = blockIdx.x;
  const int pos = min(state->pos, max_seq - 1);
  const int seq = pos + 1;
  const int chunks = (seq + kChunk - 1) / kChunk;
  if (c >= chunks) return;  // the grid covers max_seq; idle chunks exit
  const int group = heads / kv_heads;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int p0 = c * kChunk;
  const int plen = min(kChunk, seq - p0);
  const size_t head_base = static_cast<size_t>(g) * max_seq * HD;

  __shared__ float qs[kAttentionMaxGroup][HD];
  __shared__ float knew[HD];
  __shared__ __align__(16) uint16_t vt[kChunk][HD];
  __shared__ float sc[kAttentionMaxGroup][kChunk];
  __shared__ float mx[kAttentionMaxGroup], sm[kAttentionMaxGroup];
  __shared__ int last;

  // This lane's key row (raw BF16), issued first to overlap its latency.
  const int p = p0 + lane;
  const bool valid = lane < plen;
  uint4 kraw[kPieces];
  if (valid && p != pos) {
    const uint4* kr = reinterpret_cast<const uint4*>(key_cache + head_base +
                                                     static_cast<size_t>(p) * HD);
#pragma unroll
    for (int j = 0; j < kPieces; ++j) kraw[j] = kr[j];
  }
  // Stage the chunk's value rows; row pos comes from v_new.
  for (int i = tid; i < plen * kPieces; i += kThreads) {
    const int row = i / kPieces, piece = i % kPieces;
    const uint16_t* src = p0 + row == pos
                              ? v_new + static_cast<size_t>(g) * HD
                              : value_cache + head_base + static_cast<size_t>(p0 + row) * HD;
    reinterpret_cast<uint4*>(vt[row])[piece] = reinterpret_cast<const uint4*>(src)[piece];
  }
  // Rotate the group's q (rounded to BF16 as the reference's rope kernel
  // stores q) and, in the owner chunk, the new k.
  const float2* cs = rope + static_cast<size_t>(pos) * half;
  for (int j = tid; j < group * half; j += kThreads) {
    const int h = j / half, i = j % half;
    const uint16_t* qh = q + static_cast<size_t>(g * group + h) * HD;
    float a = load_bf16(qh + i), b = load_bf16(qh + i + half);
    rope_pair(a, b, cs[i]);
    qs[h][i] = bf16_to_f32(f32_to_bf16(a));
    qs[h][i + half] = bf16_to_f32(f32_to_bf16(b));
  }
  const bool owner = pos >= p0 && pos < p0 + kChunk;
  if (owner) {
    const size_t at = head_base + static_cast<size_t>(pos) * HD;
    for (int i = tid; i < half; i += kThreads) {
      const uint16_t* kh = k_new + static_cast<size_t>(g) * HD;
      float a = load_bf16(kh + i), b = load_bf16(kh + i + half);
      rope_pair(a, b, cs[i]);
      const uint16_t ka = f32_to_bf16(a), kb = f32_to_bf16(b);
      knew[i] = bf16_to_f32(ka);
      knew[i + half] = bf16_to_f32(kb);
      key_cache[at + i] = ka;
      key_cache[at + i + half] = kb;
    }
    for (int i = tid; i < HD; i += kThreads) {
      value_cache[at + i] = v_new[static_cast<size_t>(g) * HD + i];
    }
  }
  __syncthreads();

  float key[HD];
  if (valid && p != pos) {
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
      key[8 * j + 0] = bf16_lo(kraw[j].x); key[8 * j + 1] = bf16_hi(kraw[j].x);
      key[8 * j + 2] = bf16_lo(kraw[j].y); key[8 * j + 3] = bf16_hi(kraw[j].y);
      key[8 * j + 4] = bf16_lo(kraw[j].z); key[8 * j + 5] = bf16_hi(kraw[j].z);
      key[8 * j + 6] = bf16_lo(kraw[j].w); key[8 * j + 7] = bf16_hi(kraw[j].w);
    }
  } else {
#pragma unroll
    for (int d = 0; d < HD; ++d) key[d] = valid ? knew[d] : 0.0f;
  }
  const float scale = 1.0f / sqrtf(static_cast<float>(HD));
  for (int h = wave; h < group; h += kWaves) {
    float dot = 0.0f;
#pragma unroll
    for (int d = 0; d < HD; ++d) dot = fmaf(qs[h][d], key[d], dot);
    const float s = valid ? dot * scale : -INFINITY;
    float m = s;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    const float e = valid ? expf(s - m) : 0.0f;
    const float l = wave_sum(e);
    sc[h][lane] = e;
    if (lane == 0) {
      mx[h] = m;
      sm[h] = l;
    }
  }
  __syncthreads();

  // acc[r][j]: head wave + 4 r, dimension lane + 64 j.
  float acc[2][kDims];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int j = 0; j < kDims; ++j) acc[r][j] = 0.0f;
  const int h0 = wave, h1 = wave + kWaves;
#pragma unroll 4
  for (int pp = 0; pp < plen; ++pp) {
#pragma unroll
    for (int j = 0; j < kDims; ++j) {
      const float vd = bf16_to_f32(vt[pp][lane + kWave * j]);
      if (h0 < group) acc[0][j] = fmaf(sc[h0][pp], vd, acc[0][j]);
      if (h1 < group) acc[1][j] = fmaf(sc[h1][pp], vd, acc[1][j]);
    }
  }

  if (chunks == 1) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int h = wave + r * kWaves;
      if (h < group) {
#pragma unroll
        for (int j = 0; j < kDims; ++j) {
          out[static_cast<size_t>(g * group + h) * HD + lane + kWave * j] =
              f32_to_bf16(acc[r][j] / sm[h]);
        }
      }
    }
    return;
  }

  // Partial layout: [g][chunk][head][kRec] floats.
  const int max_chunks = (max_seq + kChunk - 1) / kChunk;
  float* base = partial + static_cast<size_t>(g) * max_chunks * kAttentionMaxGroup * kRec;
  float* mine = base + static_cast<size_t>(c) * kAttentionMaxGroup * kRec;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int h = wave + r * kWaves;
    if (h < group) {
#pragma unroll
      for (int j = 0; j < kDims; ++j) {
        __hip_atomic_store(mine + h * kRec + lane + kWave * j, acc[r][j], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
      if (lane == 0) {
        __hip_atomic_store(mine + h * kRec + HD, mx[h], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(mine + h * kRec + HD + 1, sm[h], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    last = __hip_atomic_fetch_add(counters + g, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           chunks - 1;
  }
  __syncthreads();
  if (!last) return;

  // Merge the chunks of every head of the group in chunk order.
  for (int h = wave; h < group; h += kWaves) {
    float m = -INFINITY;
    for (int cc = 0; cc < chunks; ++cc) {
      m = fmaxf(m, __hip_atomic_load(base + (cc * kAttentionMaxGroup + h) * kRec + HD,
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    }
    float l = 0.0f;
    float o[kDims];
#pragma unroll
    for (int j = 0; j < kDims; ++j) o[j] = 0.0f;
    for (int cc = 0; cc < chunks; ++cc) {
      const float* rec = base + (cc * kAttentionMaxGroup + h) * kRec;
      const float f = expf(
          __hip_atomic_load(rec + HD, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - m);
      l = fmaf(__hip_atomic_load(rec + HD + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), f, l);
#pragma unroll
      for (int j = 0; j < kDims; ++j) {
        o[j] = fmaf(__hip_atomic_load(rec + lane + kWave * j, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT),
                    f, o[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < kDims; ++j) {
      out[static_cast<size_t>(g * group + h) * HD + lane + kWave * j] = f32_to_bf16(o[j] / l);
    }
  }
  if (tid == 0) __hip_atomic_store(counters + g, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ----------------------------------------------------- prefill attention --

// Causal attention of count tokens (positions 0 .. count - 1, already in
// the caches): one wave per (query token, head), online softmax over the
// key positions 0 .. t in blocks of 64 (lane p scores key p of the block),
// then lane d accumulates output dimension d (and d + 64 when HD = 128).
template <int HD>
__global__ __launch_bounds__(kThreads) void attention_prefill_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ key_cache,
    const uint16_t* __restrict__ value_cache, uint16_t* __restrict__ out, int count, int heads,
    int kv_heads, int max_seq) {
  constexpr int kDims = HD / kWave;
  constexpr int kPieces = HD / 8;
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
      const uint4* kr = reinterpret_cast<const uint4*>(kbase + static_cast<size_t>(p) * HD);
      float dot = 0.0f;
#pragma unroll
      for (int j = 0; j < kPieces; ++j) {
        const uint4 w8 = kr[j];
        dot = fmaf(qv[8 * j + 0], bf16_lo(w8.x), dot);
        dot = fmaf(qv[8 * j + 1], bf16_hi(w8.x), dot);
        dot = fmaf(qv[8 * j + 2], bf16_lo(w8.y), dot);
        dot = fmaf(qv[8 * j + 3], bf16_hi(w8.y), dot);
        dot = fmaf(qv[8 * j + 4], bf16_lo(w8.z), dot);
        dot = fmaf(qv[8 * j + 5], bf16_hi(w8.z), dot);
        dot = fmaf(qv[8 * j + 6], bf16_lo(w8.w), dot);
        dot = fmaf(qv[8 * j + 7], bf16_hi(w8.w), dot);
      }
      s = dot * scale;
    }
    float bm = s;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) bm = fmaxf(bm, __shfl_xor(bm, off));
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
__global__ void set_state_kernel(ModelState* state, int token, int pos, int step) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    if (token >= 0) state->token = token;
    state->pos = pos;
    state->step = step;
  }
}

// The end of a decode step: record the token the LM head chose and move to
// the next position.
__global__ void advance_kernel(ModelState* state, int* __restrict__ history, int history_len) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    const int step = state->step;
    if (step < history_len) history[step] = state->token;
    state->step = step + 1;
    state->pos = state->pos + 1;
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

void launch_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* out, int rows, int hidden,
                     float eps, hipStream_t stream) {
  hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(kThreads), 0, stream, x, w, out, rows,
                     hidden, eps);
}

void launch_rope_store(uint16_t* q, uint16_t* k, const uint16_t* v, uint16_t* key_cache,
                       uint16_t* value_cache, const float2* rope, int count, int start,
                       int heads, int kv_heads, int head_dim, int max_seq,
                       hipStream_t stream) {
  hipLaunchKernelGGL(rope_store_kernel, dim3(count), dim3(kThreads), 0, stream, q, k, v,
                     key_cache, value_cache, rope, count, start, heads, kv_heads, head_dim,
                     max_seq);
}

bool attention_head_dim_supported(int head_dim) { return head_dim == 64 || head_dim == 128; }

int attention_decode_chunks(int max_seq) { return (max_seq + kChunk - 1) / kChunk; }

size_t attention_decode_partial_floats(int kv_heads, int head_dim, int max_seq) {
  return static_cast<size_t>(kv_heads) * attention_decode_chunks(max_seq) * kAttentionMaxGroup *
         (head_dim + 2);
}

void launch_attention_decode(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                             uint16_t* key_cache, uint16_t* value_cache, const float2* rope,
                             const ModelState* state, int heads, int kv_heads, int head_dim,
                             int max_seq, float* partial, int* counters, uint16_t* out,
                             hipStream_t stream) {
  const dim3 grid(attention_decode_chunks(max_seq), kv_heads);
  if (head_dim == 64) {
    hipLaunchKernelGGL(attention_decode_kernel<64>, grid, dim3(kThreads), 0, stream, q, k_new,
                       v_new, key_cache, value_cache, rope, state, heads, kv_heads, max_seq,
                       partial, counters, out);
  } else {
    hipLaunchKernelGGL(attention_decode_kernel<128>, grid, dim3(kThreads), 0, stream, q, k_new,
                       v_new, key_cache, value_cache, rope, state, heads, kv_heads, max_seq,
                       partial, counters, out);
  }
}

void launch_attention_prefill(const uint16_t* q, const uint16_t* key_cache,
                              const uint16_t* value_cache, uint16_t* out, int count, int heads,
                              int kv_heads, int head_dim, int max_seq, hipStream_t stream) {
  const int waves = count * heads;
  const int blocks = (waves + kThreads / kWave - 1) / (kThreads / kWave);
  if (head_dim == 64) {
    hipLaunchKernelGGL(attention_prefill_kernel<64>, dim3(blocks), dim3(kThreads), 0, stream, q,
                       key_cache, value_cache, out, count, heads, kv_heads, max_seq);
  } else {
    hipLaunchKernelGGL(attention_prefill_kernel<128>, dim3(blocks), dim3(kThreads), 0, stream, q,
                       key_cache, value_cache, out, count, heads, kv_heads, max_seq);
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

void launch_set_state(ModelState* state, int token, int pos, int step, hipStream_t stream) {
  hipLaunchKernelGGL(set_state_kernel, dim3(1), dim3(kWave), 0, stream, state, token, pos, step);
}

void launch_advance(ModelState* state, int* history, int history_len, hipStream_t stream) {
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(kWave), 0, stream, state, history,
                     history_len);
}

}  // namespace qlin
