// Prefill (M = tokens > 1) Linear kernels for gfx950: W8A16 group-64 dequant
// GEMM and BF16 GEMM on CDNA4 MFMA (v_mfma_f32_32x32x16_bf16).
//
// Both compute Y[m, n] = bf16(sum_k X[m, k] W[n, k] + bias[n]) with X
// [M, K] and W [N, K] row-major, K contiguous: the layout MFMA wants for
// both operands, so no operand is transposed anywhere.
//
// Mapping.  A workgroup of 4 waves owns a BM x BN output tile and walks K
// in stages of 64 columns — one W8A16 quantisation group.  Each stage is
// staged in LDS as BF16 (X rows and W rows, 128 bytes each), double
// buffered: the global loads of stage g + 1 are in flight while the MFMAs
// of stage g run, then written to the other buffer, one barrier per stage.
// Each wave owns a TM x TN sub-tile = FM x FN MFMA tiles of 32 x 32.
//
// W8A16.  The int8 weights are converted to BF16 while filling LDS (exact:
// |q| <= 127 needs 7 significand bits, BF16 has 8), once per workgroup and
// shared by every wave that uses those columns.  The MFMAs of a stage sum
// q * x into a per-stage FP32 partial; the group scale s[n, g] is applied to
// that partial once (acc = fma(partial, s, acc)).  So the product uses the
// exact dequantised weight q * s, as the GEMV and the CPU FP32 path do;
// the reference instead rounds q * s to BF16 before its WMMA
// (src/cuda/kernels.cu:1091).  In the 32 x 32 accumulator layout every
// value a lane holds is in one output column, so a lane needs one scale per
// MFMA tile column per stage.
//
// LDS layout.  A staged row is eight 16-byte chunks (8 BF16 each).  Chunk c
// of row r is stored at slot c ^ (r & 7): the 8 rows a group of lanes reads
// at one chunk index land in 8 different slots, i.e. all 32 banks.
//
// Reference behaviour restated (src/cuda/kernels.cu): gemm_w8a16 launcher
// 1657-1684 and its WMMA kernels 1096-1322; gemm_bf16 launcher 1600-1625 and
// kernels 605-951.  Shapes the MFMA path does not take (K % 64 != 0,
// unaligned pointers) go to the exact generic kernels, as the reference's
// dispatch sends them to linear_w8a16_kernel (1324-1387).
#include <stdint.h>

#include <algorithm>
#include <initializer_list>

#include "device_common.hpp"
#include "linear_kernels.hpp"
#include "status.hpp"

namespace qlin {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// A 16-byte LDS read the compiler does not track (the direct-X loop orders
// its reads itself: an explicit vmcnt wait and barrier before, an explicit
// lgkmcnt wait before the first use).
__device__ __forceinline__ bf16x8_t lds_read16_untracked(const uint4* p) {
  const uint32_t addr = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint4*)p));
  bf16x8_t v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 waves
constexpr int kStageK = 64;    // K columns per stage = one quantisation group
constexpr int kRowChunks = 8;  // 16-byte BF16 chunks per staged row
#ifndef QLIN_GEMM_PREFETCH
#define QLIN_GEMM_PREFETCH 2
#endif
constexpr int kPrefetch = QLIN_GEMM_PREFETCH;  // stages of loads in flight
#ifndef QLIN_GEMM_WAVES_ATTR
#define QLIN_GEMM_WAVES_ATTR
#endif

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4 v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// A raw buffer resource over [base, base + bytes): loads past the end
// return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           0x00020000);
}

__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t voffset,
                                               uint32_t soffset) {
  return __builtin_bit_cast(uint4,
                            __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, 0));
}

#ifndef QLIN_LDS_SWIZZLE
#define QLIN_LDS_SWIZZLE 1
#endif
__device__ __forceinline__ int lds_slot(int row, int chunk) {
#if QLIN_LDS_SWIZZLE == 1
  return row * kRowChunks + (chunk ^ ((row >> 1) & 7));
#else
  return row * kRowChunks + (chunk ^ (row & 7));
#endif
}

// Two small integers held exactly as FP32 -> a BF16 pair (lo in bits
// 0-15): the high halves of both words, one byte permute.
__device__ __forceinline__ uint32_t pack_hi_halves(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// 16 int8 -> 16 BF16 (two 16-byte chunks), exact: |q| <= 127 needs 7
// significand bits, BF16 has 8.
__device__ __forceinline__ void i8x16_to_bf16(const uint4 q, uint4& lo, uint4& hi) {
  lo.x = pack_hi_halves(sbyte0(q.x), sbyte1(q.x));
  lo.y = pack_hi_halves(sbyte2(q.x), sbyte3(q.x));
  lo.z = pack_hi_halves(sbyte0(q.y), sbyte1(q.y));
  lo.w = pack_hi_halves(sbyte2(q.y), sbyte3(q.y));
  hi.x = pack_hi_halves(sbyte0(q.z), sbyte1(q.z));
  hi.y = pack_hi_halves(sbyte2(q.z), sbyte3(q.z));
  hi.z = pack_hi_halves(sbyte0(q.w), sbyte1(q.w));
  hi.w = pack_hi_halves(sbyte2(q.w), sbyte3(q.w));
}

// Instruction-group order for one stage (sched_group_barrier masks: 0x008
// MFMA, 0x100 LDS read, 0x200 LDS write, 0x020 global read, 0x002 VALU).
// Each MFMA is followed by its share of the stage's remaining fragment
// reads, of the VALU work (the int8 conversion of the next stage) and of
// the next stage's LDS writes and global loads, so the matrix core stays
// busy while the rest issues.  Shares are spread evenly: group i of N gets
// total * (i + 1) / N - total * i / N.
template <int I, int N, int READS, int VALU, int WRITES, int LOADS>
struct StageSchedule {
  static __device__ __forceinline__ void emit() {
    constexpr int r = READS * (I + 1) / N - READS * I / N;
    constexpr int v = VALU * (I + 1) / N - VALU * I / N;
    constexpr int w = WRITES * (I + 1) / N - WRITES * I / N;
    constexpr int l = LOADS * (I + 1) / N - LOADS * I / N;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);
    if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x002, v, 0);
    if constexpr (w > 0) __builtin_amdgcn_sched_group_barrier(0x200, w, 0);
    if constexpr (l > 0) __builtin_amdgcn_sched_group_barrier(0x020, l, 0);
    StageSchedule<I + 1, N, READS, VALU, WRITES, LOADS>::emit();
  }
};
template <int N, int READS, int VALU, int WRITES, int LOADS>
struct StageSchedule<N, N, READS, VALU, WRITES, LOADS> {
  static __device__ __forceinline__ void emit() {}
};

// A tile reduced over part of K.  The tile's `parts` workgroups each sum
// `count` stages from `begin` and write their FP32 partial to
// partial + index * tile_floats (index = this part); the last one to finish
// (counted on *counter) adds all the parts in index order — so the result
// does not depend on which finished last — and runs the epilogue.
struct SplitK {
  int begin = 0;
  int count = 0;  // 0: the whole of K, no split
  int parts = 1;
  int index = 0;
  float* partial = nullptr;  // this tile's parts, parts * tile_floats floats
  int* counter = nullptr;
  bool xcd_local = false;    // every part of the tile runs on one XCD
  bool help = false;         // the launch's own workgroups sum the parts
};

// Split-K hand-off; returns true in the workgroup that finishes the tile
// (acc then holds the tile's full sum).  Each thread's FP32 values are
// stored as 16-byte vectors at [(i * 256 + thread) * 4], i < 4 FM FN, so a
// wave's stores and loads are contiguous.
// Coherence across XCDs without cache flushes: the parts are written and
// read with device-coherent (sc1) buffer accesses, which the AMDGPU memory
// model uses for agent-scope atomic stores and loads; every thread waits
// for its stores to complete before the barrier that precedes the arrival
// count (an agent-scope atomic), and the finishing workgroup reads the parts
// only after that count.  Nothing waits on another workgroup: the ones that
// are not last simply exit.
constexpr int kCoherent = 16;  // buffer cache policy: sc1

template <int FM, int FN, int THREADS = kThreads>
__device__ __forceinline__ bool splitk_fixup(f32x16_t (&acc)[FM][FN], const SplitK& sp) {
  constexpr int kVec = 4 * FM * FN;  // 16-byte vectors per thread
  constexpr int kTileBytes = kVec * THREADS * 16;
  __shared__ int last;
  const int tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t pr =
      make_rsrc(sp.partial, static_cast<uint32_t>(sp.parts) * kTileBytes);
  const uint32_t mine = static_cast<uint32_t>(sp.index) * kTileBytes;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i = (fm * FN + fn) * 4 + q;
        const f32x4_t v = {acc[fm][fn][4 * q], acc[fm][fn][4 * q + 1], acc[fm][fn][4 * q + 2],
                           acc[fm][fn][4 * q + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), pr,
                                               mine + (i * THREADS + tid) * 16u, 0, kCoherent);
      }
  __builtin_amdgcn_s_waitcnt(0);  // this thread's parts are stored
  __syncthreads();
  if (tid == 0) {
    last = __hip_atomic_fetch_add(sp.counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           sp.parts - 1;
  }
  __syncthreads();
  if (!last) return false;
  f32x16_t sum[FM][FN];
  for (int p = 0; p < sp.parts; ++p) {
    const uint32_t base = static_cast<uint32_t>(p) * kTileBytes;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int i = (fm * FN + fn) * 4 + q;
          f32x4_t v;
          if (p == sp.index) {
            v = f32x4_t{acc[fm][fn][4 * q], acc[fm][fn][4 * q + 1], acc[fm][fn][4 * q + 2],
                        acc[fm][fn][4 * q + 3]};
          } else {
            v = __builtin_bit_cast(
                f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                             pr, base + (i * THREADS + tid) * 16u, 0, kCoherent));
          }
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            if (p == 0) {
              sum[fm][fn][4 * q + c] = v[c];
            } else {
              sum[fm][fn][4 * q + c] += v[c];
            }
          }
        }
  }
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = sum[fm][fn];
  if (tid == 0) {  // ready for the next launch
    __hip_atomic_store(sp.counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return true;
}

template <int BM, int BN, int WAVES_M, bool W8>
struct TileShape {
  static constexpr int kWavesN = 4 / WAVES_M;
  static constexpr int TM = BM / WAVES_M;
  static constexpr int TN = BN / kWavesN;
  static constexpr int FM = TM / 32;
  static constexpr int FN = TN / 32;
  // Global 16-byte loads per thread per stage.
  static constexpr int A_LOADS = BM * kRowChunks / kThreads;
  static constexpr int B_LOADS = W8 ? BN * (kStageK / 16) / kThreads : BN * kRowChunks / kThreads;
  static_assert(WAVES_M == 1 || WAVES_M == 2 || WAVES_M == 4, "4 waves per workgroup");
  static_assert(FM >= 1 && FN >= 1 && TM % 32 == 0 && TN % 32 == 0, "32 x 32 MFMA tiles");
  static_assert(A_LOADS >= 1 && B_LOADS >= 1, "every thread loads at least one chunk");
};

// One workgroup's BM x BN tile of Y at (m0, n0) over all of K (a multiple
// of 64).  The epilogue adds the bias and writes BF16.
//
// Pipeline: the global loads of stage g + D are issued as soon as stage g
// has been written to LDS, so D stages of loads are in flight while the
// MFMAs run; a register slot per stage in flight (the loop is unrolled by
// D so every slot index is a constant).  LDS is double buffered: stage g
// is written to buffer g & 1, one barrier, then its MFMAs.  A wave that
// writes stage g + 1 into the other buffer has passed the barrier of stage
// g, which every wave reaches only after its MFMAs of stage g - 1, the
// last reader of that buffer.
template <int BM, int BN, int WAVES_M, bool W8, int D>
__device__ __forceinline__ void gemm_tile(const GemmArgs& a, int m0, int n0,
                                          const SplitK& split = SplitK{},
                                          const GemmGroupDesc* epi = nullptr) {
  using S = TileShape<BM, BN, WAVES_M, W8>;
  constexpr int FM = S::FM, FN = S::FN;
  __shared__ uint4 lds_a[2][BM * kRowChunks];
  __shared__ uint4 lds_b[2][BN * kRowChunks];
  __shared__ float lds_s[2][W8 ? BN : 1];  // W8: group scales of the stage's rows

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WAVES_M;
  const int wn = wave / WAVES_M;
  const int r = lane & 31;   // row of an A fragment / column of a B fragment
  const int h = lane >> 5;   // which half of the 64 staged columns' chunks
  const int groups = a.k / kStageK;  // scale row stride
  // This workgroup's stages: [split.begin, split.begin + stages) of the
  // K / 64 groups (all of them unless the tile is split over K).
  const int stages = split.count > 0 ? split.count : groups;
  const int sbeg = split.count > 0 ? split.begin : 0;

  // ---- global -> register staging, one slot per stage in flight ----
  // Buffer loads: a row past M or N is out of the resource's range and
  // reads as zero, so the loads need no branches (the host checks that
  // every operand fits a 32-bit byte offset).  Each thread's byte offsets
  // are fixed; the stage's column offset is a scalar (soffset), clamped to
  // the last stage so that loads issued past it stay inside the tensor.
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, static_cast<uint32_t>(a.m) * a.k * 2u);
  const __amdgpu_buffer_rsrc_t wr =
      make_rsrc(a.w, static_cast<uint32_t>(a.n) * a.k * (W8 ? 1u : 2u));
  uint32_t xoff[S::A_LOADS], woff[S::B_LOADS];
#pragma unroll
  for (int i = 0; i < S::A_LOADS; ++i) {
    const int c = tid + kThreads * i;
    xoff[i] = ((static_cast<uint32_t>(m0) + (c >> 3)) * a.k + (c & 7) * 8) * 2u;
  }
#pragma unroll
  for (int i = 0; i < S::B_LOADS; ++i) {
    const int c = tid + kThreads * i;
    woff[i] = W8 ? (static_cast<uint32_t>(n0) + (c >> 2)) * a.k + (c & 3) * 16
                 : ((static_cast<uint32_t>(n0) + (c >> 3)) * a.k + (c & 7) * 8) * 2u;
  }
  // W8: the scales of row n0 + tid % BN (clamped into the tensor; rows past
  // N are never used) for every stage.
  const uint16_t* srow = W8 ? a.s + static_cast<size_t>(min(n0 + tid % BN, a.n - 1)) * groups
                            : nullptr;
  uint4 ra[D][S::A_LOADS];
  uint4 rb[D][S::B_LOADS];
  uint32_t rs[D];  // W8: the group scale of row n0 + tid % BN of the stage

  auto load_stage = [&](int g, uint4 (&xa)[S::A_LOADS], uint4 (&xb)[S::B_LOADS],
                        uint32_t& xs) {
    const uint32_t gc = static_cast<uint32_t>(min(g, stages - 1) + sbeg);
    const uint32_t kbyte = gc * kStageK * 2u;
#pragma unroll
    for (int i = 0; i < S::A_LOADS; ++i) xa[i] = buffer_load16(xr, xoff[i], kbyte);
#pragma unroll
    for (int i = 0; i < S::B_LOADS; ++i)
      xb[i] = buffer_load16(wr, woff[i], W8 ? gc * kStageK : kbyte);
    // A 16-bit global load zero-extends in the load itself.
    if (W8) xs = gload(srow + gc);
  };

  auto store_stage = [&](int buf, const uint4 (&xa)[S::A_LOADS],
                         const uint4 (&xb)[S::B_LOADS], uint32_t xs) {
    // Threads tid and tid + BN hold the same row's scale: both write it,
    // which keeps the fill free of branches.
    if (W8) lds_s[buf][tid % BN] = bf16_to_f32(xs);
#pragma unroll
    for (int i = 0; i < S::A_LOADS; ++i) {
      const int c = tid + kThreads * i;
      lds_a[buf][lds_slot(c >> 3, c & 7)] = xa[i];
    }
#pragma unroll
    for (int i = 0; i < S::B_LOADS; ++i) {
      const int c = tid + kThreads * i;
      if (W8) {
        const int row = c >> 2, col = c & 3;
        uint4 lo, hi;
        i8x16_to_bf16(xb[i], lo, hi);
        lds_b[buf][lds_slot(row, 2 * col)] = lo;
        lds_b[buf][lds_slot(row, 2 * col + 1)] = hi;
      } else {
        lds_b[buf][lds_slot(c >> 3, c & 7)] = xb[i];
      }
    }
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[fm][fn][e] = 0.0f;

  // Stage g's MFMAs on LDS buffer buf.  Lane (r, h) multiplies k-chunks
  // 4h .. 4h + 3 of the stage, one per MFMA k-step; A and B fragments use
  // the same chunk, so their k slots agree.
  auto compute_stage = [&](int buf) {
    // All fragments of the stage are read first (distinct registers), so
    // the LDS latency is paid once per stage instead of once per k-step.
    bf16x8_t fa[4][FM], fb[4][FN];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int chunk = 4 * h + ks;
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        fa[ks][fm] = as_bf16x8(lds_a[buf][lds_slot(wm * S::TM + fm * 32 + r, chunk)]);
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
        fb[ks][fn] = as_bf16x8(lds_b[buf][lds_slot(wn * S::TN + fn * 32 + r, chunk)]);
    }
    float sc[FN];
    if (W8) {
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) sc[fn] = lds_s[buf][wn * S::TN + fn * 32 + r];
    }
    f32x16_t part[FM][FN];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          if (W8) {
            const f32x16_t zero = {};
            part[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                fa[ks][fm], fb[ks][fn], ks == 0 ? zero : part[fm][fn], 0, 0, 0);
          } else {
            acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[ks][fm], fb[ks][fn],
                                                                  acc[fm][fn], 0, 0, 0);
          }
        }
      }
    }
    if (W8) {
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            acc[fm][fn][e] = fmaf(part[fm][fn][e], sc[fn], acc[fm][fn][e]);
      }
    }
  };

  // Pipeline order of one main-loop stage (see StageSchedule): the k-step 0
  // fragments (and the W8 scales) first, the k-step 1..3 fragments spread
  // over the first three quarters of the MFMAs, the next stage's int8
  // conversion, LDS writes and global loads over all of them.
  auto schedule_stage = [&]() {
    constexpr int kMfma = 4 * FM * FN;
    constexpr int kFirstReads = FM + FN + (W8 ? FN : 0);
    constexpr int kLaterReads = 3 * (FM + FN);
    constexpr int kValu = W8 ? 24 * S::B_LOADS : 0;
    constexpr int kWrites = S::A_LOADS + (W8 ? 2 : 1) * S::B_LOADS + (W8 ? 1 : 0);
    constexpr int kLoads = S::A_LOADS + S::B_LOADS + (W8 ? 1 : 0);
    __builtin_amdgcn_sched_group_barrier(0x100, kFirstReads, 0);
    StageSchedule<0, kMfma, kLaterReads * 4 / 3, kValu, kWrites, kLoads>::emit();
  };

  // Stage g lives in register slot g % D and LDS buffer g & 1.  Iteration
  // g runs the MFMAs of stage g and, in the same instruction stream, writes
  // stage g + 1 into the other LDS buffer and issues the loads of stage
  // g + 1 + D; one barrier ends the iteration.  The other buffer's last
  // reader was stage g - 1, finished by every wave before the previous
  // barrier.  With D even, full rounds of D stages have compile-time
  // buffer indices, so the compiler sees the writes and the MFMA reads
  // touch different LDS arrays and can interleave them.  Loads past the
  // last stage (issued by the last full round) read in-range neighbouring
  // bytes or zeros and are never stored.
  static_assert(D % 2 == 0, "full rounds keep the LDS buffer parity");
#pragma unroll
  for (int j = 0; j < D; ++j) load_stage(j, ra[j], rb[j], rs[j]);
  store_stage(0, ra[0], rb[0], rs[0]);
  load_stage(D, ra[0], rb[0], rs[0]);
  __syncthreads();

  int g0 = 0;
  for (; g0 + D < stages; g0 += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int g = g0 + j;
      compute_stage(j & 1);
      const int jn = (j + 1) % D;
      store_stage((j + 1) & 1, ra[jn], rb[jn], rs[jn]);
      load_stage(g + 1 + D, ra[jn], rb[jn], rs[jn]);
      schedule_stage();
      __syncthreads();
    }
  }
  // The last 1..D stages: stage g0 is in LDS buffer 0, later ones in
  // register slots 1.. (no further loads).
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const int g = g0 + j;
    if (g < stages) {
      compute_stage(j & 1);
      if (g + 1 < stages) store_stage((j + 1) & 1, ra[(j + 1) % D], rb[(j + 1) % D], rs[(j + 1) % D]);
      __syncthreads();
    }
  }

  if (split.parts > 1 && !splitk_fixup<FM, FN>(acc, split)) return;

  if constexpr (BM == 64 && BN == 64) {
    if (epi && epi->rope_kind != 0) {
      // The q|k|v epilogue (GemmGroupDesc::rope_kind): the tile's BF16 rows
      // staged as floats in the stage buffers, then each thread one row's
      // 8 rotation pairs (or 16 values of v), the arithmetic of
      // rope_store_rows_kernel on the same BF16 values.
      float* ep = reinterpret_cast<float*>(&lds_a[0][0]);  // 64 x 64 floats
      static_assert(sizeof(lds_a) == 64 * 64 * sizeof(float), "the staged tile fits");
      __syncthreads();  // every wave's last fragment reads are done
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int cl = wn * S::TN + fn * 32 + r;
        const int n = n0 + cl;
        const float b = a.bias && n < a.n ? bf16_to_f32(gload(a.bias + n)) : 0.0f;
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int rl = wm * S::TM + fm * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
            ep[rl * 64 + cl] = bf16_to_f32(f32_to_bf16(acc[fm][fn][e] + b));
          }
        }
      }
      __syncthreads();
      const int rl = tid >> 2, m = m0 + rl, pos = epi->rope_start + m;
      if (m >= a.m || pos >= epi->max_seq || n0 + 64 > a.n) return;
      const float* er = ep + rl * 64;
      uint16_t* cache_row =
          epi->kv_cache ? epi->kv_cache + (static_cast<size_t>(n0 / 64) * epi->max_seq + pos) * 64
                        : nullptr;
      if (epi->rope_kind == 3) {
        const int c0 = (tid & 3) * 16;
        uint32_t w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = pack2_bf16(er[c0 + 2 * j], er[c0 + 2 * j + 1]);
        store_global16(cache_row + c0, make_uint4(w[0], w[1], w[2], w[3]));
        store_global16(cache_row + c0 + 8, make_uint4(w[4], w[5], w[6], w[7]));
        return;
      }
      const int c0 = (tid & 3) * 8;
      const float2* cs = epi->rope + static_cast<size_t>(pos) * 32 + c0;
      float lo[8], hi[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        lo[j] = er[c0 + j];
        hi[j] = er[c0 + 32 + j];
        rope_pair(lo[j], hi[j], cs[j]);
      }
      const uint4 wl = make_uint4(pack2_bf16(lo[0], lo[1]), pack2_bf16(lo[2], lo[3]),
                                  pack2_bf16(lo[4], lo[5]), pack2_bf16(lo[6], lo[7]));
      const uint4 wh = make_uint4(pack2_bf16(hi[0], hi[1]), pack2_bf16(hi[2], hi[3]),
                                  pack2_bf16(hi[4], hi[5]), pack2_bf16(hi[6], hi[7]));
      uint16_t* dst = epi->rope_kind == 1 ? a.y + static_cast<size_t>(m) * a.n + n0 : cache_row;
      store_global16(dst + c0, wl);
      store_global16(dst + 32 + c0, wh);
      return;
    }
  }

  // ---- epilogue: accumulator element e of a 32 x 32 tile is at row
  // 8 (e / 4) + 4 h + e % 4, column r ----
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
    const int n = n0 + wn * S::TN + fn * 32 + r;
    if (n >= a.n) continue;
    const float b = a.bias ? bf16_to_f32(gload(a.bias + n)) : 0.0f;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * S::TM + fm * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (m < a.m) gstore(a.y + static_cast<size_t>(m) * a.n + n, f32_to_bf16(acc[fm][fn][e] + b));
      }
    }
  }
}

// ------------------------------------------------------------------------
// Wide tile: 256 x 128 of Y per workgroup of 8 waves (512 threads), for M
// of a few hundred rows and more.
//
// Why this shape on gfx950.  The MFMA pipe of a SIMD needs two waves to
// stay busy while one of them waits on LDS, so 8 waves share the CU; each
// wave owns a 64 x 64 block (2 x 2 tiles of 32 x 32, waves 4 along M x 2
// along N).  LDS traffic is what bounds a stage here (the fill of a stage is
// not overlapped with the fragment reads), and the fill bytes per FLOP fall
// with the tile size: 256 x 128 moves (256 + 128) x 128 B per 4.2 MFLOP.
// With 256 rows the W8A16 int8 -> BF16 conversion is done once per weight
// element per 256 rows.
//
// LDS rows are padded to 9 chunks of 16 B: the 8 rows that lanes read at one
// chunk index land in 8 different bank groups, and the k-step index of a
// fragment read is an immediate offset.  Two buffers of X (256 rows) and W
// (128 rows): 108 KB.
//
// Per stage each wave computes four 4-MFMA chains (one per 32 x 32 tile,
// k-steps 0..3); under W8A16 each chain starts from zero and is folded into
// the accumulator with the group scale while the next chain runs, so the
// product is the exact dequantised q * s, as in gemm_tile.
constexpr int kWideThreads = 512;
constexpr int kWideRows = 256;
constexpr int kWideCols = 128;
constexpr int kWideRowStride = 9;  // 16-byte chunks per padded LDS row
// Epilogue staging row (floats): 128 columns + 8 pad, so the two row groups a
// wave writes at once (rows r and r + 4) fall in disjoint banks.
constexpr int kWideEpStride = kWideCols + 8;
constexpr int kWideLdsChunks =
    (2 * (kWideRows + kWideCols) * kWideRowStride > kWideRows * kWideEpStride / 4)
        ? 2 * (kWideRows + kWideCols) * kWideRowStride
        : kWideRows * kWideEpStride / 4;

// 16-byte non-temporal global store.  Results and split-K parts are read
// by the next launch, not by this one; streaming them out of L2 as they are
// written leaves less dirty data for the write-back at the end of the
// kernel (measured: 30.8 -> 28.9 us for the M = 512 layer plan).
__device__ __forceinline__ void store_nt16(void* p, u32x4 v) {
  __builtin_nontemporal_store(v, (QLIN_GLOBAL u32x4*)(p));
}

// 8 int8 -> 8 BF16 (one 16-byte chunk), exact.
__device__ __forceinline__ uint4 i8x8_to_bf16(const uint2 q) {
  uint4 o;
  o.x = pack_hi_halves(sbyte0(q.x), sbyte1(q.x));
  o.y = pack_hi_halves(sbyte2(q.x), sbyte3(q.x));
  o.z = pack_hi_halves(sbyte0(q.y), sbyte1(q.y));
  o.w = pack_hi_halves(sbyte2(q.y), sbyte3(q.y));
  return o;
}

__device__ __forceinline__ uint2 buffer_load8(__amdgpu_buffer_rsrc_t r, uint32_t voffset,
                                              uint32_t soffset) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, voffset, soffset, 0));
}

// The up_proj half of a gate|up pair tile (null w2: a plain tile).
struct WidePair {
  const void* w2 = nullptr;
  const uint16_t* s2 = nullptr;
  const uint16_t* bias2 = nullptr;
};

// Timeline slots of one workgroup (gemm_wide_grouped_timeline_kernel), in
// 100 MHz s_memrealtime ticks unless noted.
enum WideStamp {
  kStampEntry = 0,      // first instruction
  kStampLoop = 1,       // first stage in LDS (end of the prologue)
  kStampEpilogue = 2,   // last stage's MFMAs issued (start of the epilogue)
  kStampEnd = 3,        // every thread's stores done
  kStampXcc = 4,        // XCC_ID hardware register (the XCD)
  kStampHwId = 5,       // HW_ID hardware register (CU, SIMD, shader engine)
  kStampUnit = 6,       // logical block | stages << 16 | kind << 24 (0 whole, 1 part, 2 pair)
  kStampCycles = 7,     // s_memtime (shader clock) from entry to end
  kStampStored = 8,     // split part: its FP32 tile stored (in-launch hand-off)
  kStampArrived = 9,    // split part: every part has arrived (or the wait ended)
  kStampReduced = 10,   // split part: its slices summed and stored
  kStampHelp = 11,      // own unit done, the in-launch reduction (map.help) begins
  kStampSlots = 16
};

// Split-K hand-off of a wide tile inside its launch.  The tile's `parts`
// workgroups each store their FP32 tile row-major (256 x 128) at
// partial + index * 32768 floats with device-coherent (sc1) stores, wait for
// them, and count themselves on ctr[0].  Row slice s (rows s * R .. s * R +
// R - 1, R = ceil(256 / parts)) of the output is then summed over the parts
// in index order — the arithmetic of splitk_reduce_block, so the result does
// not depend on which part finished when — plus the bias, and written as
// BF16, by the workgroup that claims it (bit s of ctr[1], an agent-scope
// atomic).  A part waits, a bounded number of polls, for every part to
// arrive and then claims its own slice; the last to arrive claims its own
// and then every slice still unclaimed.  So each slice is summed exactly
// once, and no workgroup waits without end even if some part is not
// resident: a part that gives up leaves its slice to the last arrival.  The
// last of the parts to leave (ctr[2]) sets ctr[0..2] back to zero for the
// next launch.  parts <= 32.
// kLocal (build option QLIN_HANDOFF_L2, on launches whose block map puts
// every part of a tile on one XCD): the partial tiles go through that XCD's
// L2 with plain stores and loads — a part's stores have reached the L2 when
// its wait for them ends, before it counts itself, and the loads after the
// arrival count miss the CU's L1, which never held those lines — with the
// counters still agent-scope atomics.
constexpr int kWideArrivePolls = 1 << 16;
#ifndef QLIN_HANDOFF_FENCE
#define QLIN_HANDOFF_FENCE 0
#endif
#ifndef QLIN_HANDOFF_L2
#define QLIN_HANDOFF_L2 0
#endif
// X tiles of the wide tile loaded straight into LDS (buffer_load ... lds).
#ifndef QLIN_WIDE_DIRECT_A
#define QLIN_WIDE_DIRECT_A 0
#endif

template <bool kLocal>
__device__ __forceinline__ void wide_split_handoff(const GemmArgs& a, int m0, int n0,
                                                   const SplitK& sp, const uint4* tile_lds,
                                                   unsigned long long* stamp) {
  constexpr int BM = kWideRows, BN = kWideCols, NT = kWideThreads;
  constexpr bool kFence = !kLocal && QLIN_HANDOFF_FENCE;
  constexpr int kPolicy = kLocal || QLIN_HANDOFF_FENCE ? 0 : kCoherent;
  constexpr int kChunksPerRow = BN / 8;
  constexpr uint32_t kTileBytes = BM * BN * 4;
  __shared__ int shared_word;
  const int tid = threadIdx.x;
  const __amdgpu_buffer_rsrc_t pr =
      make_rsrc(sp.partial, static_cast<uint32_t>(sp.parts) * kTileBytes);
  const int c8 = (tid % kChunksPerRow) * 8;
  {
    const uint32_t mine = static_cast<uint32_t>(sp.index) * kTileBytes;
#pragma unroll
    for (int i = 0; i < BM * kChunksPerRow / NT; ++i) {
      const int row = (tid + NT * i) / kChunksPerRow;
      const int idx = row * (kWideEpStride / 4) + c8 / 4;
      const uint32_t off = mine + static_cast<uint32_t>(row * BN + c8) * 4u;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, tile_lds[idx]), pr, off, 0,
                                             kPolicy);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, tile_lds[idx + 1]), pr,
                                             off + 16u, 0, kPolicy);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this thread's part is stored
  if constexpr (kFence) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  int* ctr = sp.counter;
  if (stamp && tid == 0) stamp[kStampStored] = __builtin_amdgcn_s_memrealtime();
  if (tid == 0) {
    const int before =
        __hip_atomic_fetch_add(&ctr[0], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int state = 2;  // 2: last to arrive, 1: all arrived, 0: gave up waiting
    if (before != sp.parts - 1) {
      state = 0;
      for (int poll = 0; poll < kWideArrivePolls; ++poll) {
        if (__hip_atomic_load(&ctr[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= sp.parts) {
          state = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    shared_word = state;
  }
  __syncthreads();
  const int state = shared_word;
  if constexpr (kFence) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  if (stamp && tid == 0) stamp[kStampArrived] = __builtin_amdgcn_s_memrealtime();
  const int rows = (BM + sp.parts - 1) / sp.parts;
  const bool vec = (a.n % 8) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15u) == 0;
  const int n = n0 + c8;
  auto claim = [&](int slice) {
    __syncthreads();  // shared_word is free again
    if (tid == 0) {
      const int bit = 1 << slice;
      shared_word = (__hip_atomic_fetch_or(&ctr[1], bit, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT) & bit) == 0;
    }
    __syncthreads();
    return shared_word != 0;
  };
  auto reduce_slice = [&](int slice) {
    const int r_begin = slice * rows, r_end = min(BM, r_begin + rows);
    for (int r0 = r_begin; r0 < r_end; r0 += NT / kChunksPerRow) {
      const int row = r0 + tid / kChunksPerRow;
      const int m = m0 + row;
      if (row >= r_end || m >= a.m || n >= a.n) continue;
      const uint32_t off = static_cast<uint32_t>(row * BN + c8) * 4u;
      constexpr int kBatch = 4;  // a batch's loads are all issued before its adds
      float f[8];
      for (int p0 = 0; p0 < sp.parts; p0 += kBatch) {
        u32x4 v[kBatch][2];
#pragma unroll
        for (int q = 0; q < kBatch; ++q) {
          if (p0 + q < sp.parts) {
            const uint32_t po = static_cast<uint32_t>(p0 + q) * kTileBytes + off;
            v[q][0] = __builtin_amdgcn_raw_buffer_load_b128(pr, po, 0, kPolicy);
            v[q][1] = __builtin_amdgcn_raw_buffer_load_b128(pr, po + 16u, 0, kPolicy);
          }
        }
#pragma unroll
        for (int q = 0; q < kBatch; ++q) {
          if (p0 + q < sp.parts) {
            const float g[8] = {__uint_as_float(v[q][0].x), __uint_as_float(v[q][0].y),
                                __uint_as_float(v[q][0].z), __uint_as_float(v[q][0].w),
                                __uint_as_float(v[q][1].x), __uint_as_float(v[q][1].y),
                                __uint_as_float(v[q][1].z), __uint_as_float(v[q][1].w)};
#pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = (p0 + q) == 0 ? g[j] : f[j] + g[j];
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (a.bias && n + j < a.n) f[j] += bf16_to_f32(gload(a.bias + n + j));
      }
      uint16_t* dst = a.y + static_cast<size_t>(m) * a.n + n;
      if (vec) {
        store_nt16(dst, u32x4{pack2_bf16(f[0], f[1]), pack2_bf16(f[2], f[3]),
                              pack2_bf16(f[4], f[5]), pack2_bf16(f[6], f[7])});
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (n + j < a.n) gstore(dst + j, f32_to_bf16(f[j]));
        }
      }
    }
  };
  if (state >= 1 && claim(sp.index)) reduce_slice(sp.index);
  if (state == 2) {
    for (int s = 0; s < sp.parts; ++s) {
      if (s != sp.index && claim(s)) reduce_slice(s);
    }
  }
  __syncthreads();
  if (stamp && tid == 0) stamp[kStampReduced] = __builtin_amdgcn_s_memrealtime();
  if (tid == 0 &&
      __hip_atomic_fetch_add(&ctr[2], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
          sp.parts - 1) {
    // every part has left: ready for the next launch
    __hip_atomic_store(&ctr[0], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&ctr[1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&ctr[2], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// A plain tile covers columns n0 .. n0 + 127 of Y.  A pair tile (pair.w2
// set, a.n the pair's width) covers rows n0 .. n0 + 63 of a.w (gate) in
// its columns 0-63 and the same rows of pair.w2 (up) in columns 64-127, and
// writes columns n0 .. n0 + 63 of Y = bf16(silu(bf16(gate)) * bf16(up)),
// the arithmetic of silu_mul_kernel on the two GEMMs' BF16 outputs.
template <bool W8>
__device__ __forceinline__ void gemm_wide_tile(const GemmArgs& a, int m0, int n0,
                                               const SplitK& split = SplitK{},
                                               const WidePair& pair = WidePair{},
                                               unsigned long long* stamp = nullptr) {
  constexpr int BM = kWideRows, BN = kWideCols, NT = kWideThreads, RS = kWideRowStride;
  constexpr int A_LD = BM * kRowChunks / NT;  // X chunks per thread per stage (4)
  constexpr int B_LD = BN * kRowChunks / NT;  // W chunks per thread per stage (2)
  // LDS: the two stage buffers of X and W; after the main loop the same
  // bytes stage the FP32 tile for the epilogue.  With QLIN_WIDE_DIRECT_A the
  // X rows are unpadded (AS = 8 chunks), chunk c of row R at chunk
  // c ^ ((R >> 1) & 7): each 16-lane group of a fragment read (16 rows, one
  // chunk) then covers all 64 banks once.
#if QLIN_WIDE_DIRECT_A
  constexpr int AS = kRowChunks;
  constexpr int ABUFS = 3;  // X loaded two stages ahead
#else
  constexpr int AS = RS;
  constexpr int ABUFS = 2;
#endif
  static_assert(ABUFS * BM * AS + 2 * BN * RS <= kWideLdsChunks, "stage buffers fit");
  __shared__ uint4 lds_raw[kWideLdsChunks];
  uint4 (*lds_a)[BM * AS] = reinterpret_cast<uint4 (*)[BM * AS]>(lds_raw);
  uint4 (*lds_b)[BN * RS] = reinterpret_cast<uint4 (*)[BN * RS]>(lds_raw + ABUFS * BM * AS);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 3, wn = wave >> 2;
  const int r = lane & 31, h = lane >> 5;
  const int groups = a.k / kStageK;  // scale row stride
  const int stages = split.count > 0 ? split.count : groups;
  const int sbeg = split.count > 0 ? split.begin : 0;

  // Branch-free buffer loads as in gemm_tile: rows past M or N read zero.
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, static_cast<uint32_t>(a.m) * a.k * 2u);
  const bool paired = pair.w2 != nullptr;
  const uint32_t wbytes = static_cast<uint32_t>(a.n) * a.k * (W8 ? 1u : 2u);
  const uint32_t sbytes = W8 ? static_cast<uint32_t>(a.n) * groups * 2u : 0u;
  // W rows 0-63 of the tile come from wr, rows 64-127 from wr_hi: the same
  // tensor 64 rows on for a plain tile, up_proj's same rows for a pair.
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(a.w, wbytes);
  const __amdgpu_buffer_rsrc_t wr_hi = paired ? make_rsrc(pair.w2, wbytes) : wr;
  // The scales of this wave's columns (wave-uniform: waves 4-7 hold
  // columns 64-127).
  const bool hi_wave = __builtin_amdgcn_readfirstlane(wn) == 1;
  const __amdgpu_buffer_rsrc_t sr =
      make_rsrc(paired && hi_wave ? pair.s2 : a.s, sbytes);
  const int col0 = paired ? n0 : n0 + wn * 64;  // W row of this wave's first column
  uint32_t xoff[A_LD], woff[B_LD];
#pragma unroll
  for (int i = 0; i < A_LD; ++i) {
    const int c = tid + NT * i;
    xoff[i] = ((static_cast<uint32_t>(m0) + (c >> 3)) * a.k + (c & 7) * 8) * 2u;
  }
#pragma unroll
  for (int i = 0; i < B_LD; ++i) {
    const int c = tid + NT * i;  // W row (c >> 3) of the tile: 64 i .. 64 i + 63
    const int row = paired ? n0 + (c >> 3) - 64 * i : n0 + (c >> 3);
    woff[i] = ((static_cast<uint32_t>(row)) * a.k + (c & 7) * 8) * (W8 ? 1u : 2u);
  }
  static_assert(B_LD == 2, "W rows 0-63 and 64-127 of the tile: one load each");
  // W8: scale rows of this lane's two output columns
  uint32_t soff[2];
#pragma unroll
  for (int fn = 0; fn < 2; ++fn)
    soff[fn] = (static_cast<uint32_t>(col0 + fn * 32 + r) * groups) * 2u;
  const int fb_base[2] = {(wn * 64 + r) * RS + 4 * h, (wn * 64 + 32 + r) * RS + 4 * h};
  // X fragment chunk ks of row group fm: row wm * 64 + 32 fm + r, chunk 4 h + ks
  int fa[2][4];
#pragma unroll
  for (int fm = 0; fm < 2; ++fm) {
    const int row = wm * 64 + 32 * fm + r;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#if QLIN_WIDE_DIRECT_A
      fa[fm][ks] = row * AS + ((4 * h + ks) ^ ((row >> 1) & 7));
#else
      fa[fm][ks] = row * AS + 4 * h + ks;
#endif
    }
  }
#if QLIN_WIDE_DIRECT_A
  // Direct X fill: wave w writes stage-buffer chunks (4 w + i) * 64 + lane,
  // i < 4 (row R = chunk / 8, the chunk's swizzled place), loading the X
  // chunk that belongs there; rows past M read zero.
  uint32_t xdir[A_LD];
#pragma unroll
  for (int i = 0; i < A_LD; ++i) {
    const int slot = (wave * A_LD + i) * 64 + lane;
    const int row = slot >> 3;
    const int c = (slot & 7) ^ ((row >> 1) & 7);
    xdir[i] = ((static_cast<uint32_t>(m0) + row) * a.k + c * 8) * 2u;
  }
  auto load_a_direct = [&](int g, int buf) {
    const uint32_t gc = static_cast<uint32_t>(min(g, stages - 1) + sbeg);
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xr, (__attribute__((address_space(3))) void*)(&lds_a[buf][(wave * A_LD + i) * 64]), 16,
          xdir[i], gc * kStageK * 2u, 0, 0);
    }
  };
  static_assert(A_LD * 64 * (NT / 64) == BM * kRowChunks, "one stage of X: A_LD loads a lane");
#endif

  // Global -> register staging, one slot per stage in flight (2).
  struct Slot {
    uint4 a[A_LD];
    uint4 b[W8 ? 1 : B_LD];  // BF16 W
    uint2 q[W8 ? B_LD : 1];  // int8 W
  };
  Slot sl[2];
  auto load = [&](int g, Slot& d) {
    const uint32_t gc = static_cast<uint32_t>(min(g, stages - 1) + sbeg);
#if !QLIN_WIDE_DIRECT_A
#pragma unroll
    for (int i = 0; i < A_LD; ++i) d.a[i] = buffer_load16(xr, xoff[i], gc * kStageK * 2u);
#endif
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      if (W8) {
        d.q[i] = buffer_load8(i == 0 ? wr : wr_hi, woff[i], gc * kStageK);
      } else {
        d.b[i] = buffer_load16(i == 0 ? wr : wr_hi, woff[i], gc * kStageK * 2u);
      }
    }
  };
  // W8: the group scales of stage g, loaded one stage ahead
  // (the direct-X loop keeps scales as loaded, 16 bits, until folded: a
  // conversion at load time would wait for the X loads issued after them)
#if QLIN_WIDE_DIRECT_A
  using ScaleT = uint16_t;
#else
  using ScaleT = uint32_t;
#endif
  auto load_scales = [&](int g, ScaleT (&xs)[2]) {
    if (W8) {
      const uint32_t gc = static_cast<uint32_t>(min(g, stages - 1) + sbeg);
#pragma unroll
      for (int fn = 0; fn < 2; ++fn) {
        xs[fn] = __builtin_amdgcn_raw_buffer_load_b16(sr, soff[fn], gc * 2u, 0);
      }
    }
  };
  auto store = [&](int buf, const Slot& d) {
#if !QLIN_WIDE_DIRECT_A
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int c = tid + NT * i;
      lds_a[buf][(c >> 3) * RS + (c & 7)] = d.a[i];
    }
#endif
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int c = tid + NT * i;
      lds_b[buf][(c >> 3) * RS + (c & 7)] = W8 ? i8x8_to_bf16(d.q[i]) : d.b[i];
    }
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  typedef bf16x8_t Frag[4];  // k-steps 0..3 of one 32-row fragment
  auto chain = [&](const Frag& fa, const Frag& fb, f32x16_t& c, bool fresh) {
    const f32x16_t zero = {};
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[0], fb[0], fresh ? zero : c, 0, 0, 0);
#pragma unroll
    for (int ks = 1; ks < 4; ++ks) {
      c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[ks], fb[ks], c, 0, 0, 0);
    }
  };
  auto fold = [&](f32x16_t& dst, const f32x16_t& p, ScaleT s) {
    const float sc = bf16_to_f32(static_cast<uint32_t>(s));
#pragma unroll
    for (int e = 0; e < 16; ++e) dst[e] = fmaf(p[e], sc, dst[e]);
  };
  // Stage on LDS buffer buf with scales cs; loads stage sg's scales into ns;
  // the store of the next stage (slot sd into buffer nbuf) and the loads of
  // stage lg (into slot sd) ride in the MFMA stream.
  // abuf: the X buffer of this stage; with QLIN_WIDE_DIRECT_A, X of stage
  // sg + 1 (if dma) goes into X buffer dbuf.
  auto compute = [&](int buf, const ScaleT (&cs)[2], ScaleT (&ns)[2], int sg, bool st,
                     int nbuf, Slot* sd, bool ld, int lg, int abuf, bool dma, int dbuf) {
    load_scales(sg, ns);
    Frag A0, A1, B0, B1;
#if QLIN_WIDE_DIRECT_A
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      A0[ks] = lds_read16_untracked(&lds_a[abuf][fa[0][ks]]);
      B0[ks] = lds_read16_untracked(&lds_b[buf][fb_base[0] + ks]);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) B1[ks] = lds_read16_untracked(&lds_b[buf][fb_base[1] + ks]);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) A1[ks] = lds_read16_untracked(&lds_a[abuf][fa[1][ks]]);
#else
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      A0[ks] = as_bf16x8(lds_a[abuf][fa[0][ks]]);
      B0[ks] = as_bf16x8(lds_b[buf][fb_base[0] + ks]);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) B1[ks] = as_bf16x8(lds_b[buf][fb_base[1] + ks]);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) A1[ks] = as_bf16x8(lds_a[abuf][fa[1][ks]]);
#endif
#if QLIN_WIDE_DIRECT_A
    // W of stage sg into the other W buffer (free since the last barrier),
    // then X of stage sg + 1 straight into the X buffer read two stages ago,
    // so no LDS write of this iteration waits behind those loads
    if (st) store(nbuf, *sd);
    __builtin_amdgcn_sched_barrier(0);
    if (dma) load_a_direct(sg + 1, dbuf);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the fragments are in
    __builtin_amdgcn_sched_barrier(0);
    if (W8) {
      f32x16_t p0, p1, p2, p3;
      chain(A0, B0, p0, true);
      chain(A0, B1, p1, true);
      chain(A1, B0, p2, true);
      fold(acc[0][0], p0, cs[0]);
      if (ld) load(lg, *sd);
      chain(A1, B1, p3, true);
      fold(acc[0][1], p1, cs[1]);
      fold(acc[1][0], p2, cs[0]);
      fold(acc[1][1], p3, cs[1]);
    } else {
      chain(A0, B0, acc[0][0], false);
      chain(A0, B1, acc[0][1], false);
      chain(A1, B0, acc[1][0], false);
      if (ld) load(lg, *sd);
      chain(A1, B1, acc[1][1], false);
    }
    return;
#endif
    if (W8) {
      // four partials, each folded once the next chain is issued: no chain
      // waits for a fold to release its registers (measured: 1.147 -> 1.12-1.13
      // us per stage, layer plan -2 % against two partials reused)
      f32x16_t p0, p1, p2, p3;
      chain(A0, B0, p0, true);
      chain(A0, B1, p1, true);
      if (st) store(nbuf, *sd);
      chain(A1, B0, p2, true);
      fold(acc[0][0], p0, cs[0]);
      if (ld) load(lg, *sd);
      chain(A1, B1, p3, true);
      fold(acc[0][1], p1, cs[1]);
      fold(acc[1][0], p2, cs[0]);
      fold(acc[1][1], p3, cs[1]);
    } else {
      chain(A0, B0, acc[0][0], false);
      chain(A0, B1, acc[0][1], false);
      if (st) store(nbuf, *sd);
      chain(A1, B0, acc[1][0], false);
      if (ld) load(lg, *sd);
      chain(A1, B1, acc[1][1], false);
    }
  };

  // Stage g: LDS buffer g & 1, register slot g & 1.  Iteration g computes
  // stage g, stores stage g + 1 (slot (g + 1) & 1, loaded two iterations
  // ago) into the other buffer — last read in iteration g - 1, before the
  // barrier that ended it — and reloads slot g & 1 with stage g + 2.  The
  // main loop is unrolled by two so buffer and slot indices are constants
  // and the vmcnt waits the compiler derives stay partial.
  ScaleT csa[2] = {0u, 0u}, csb[2] = {0u, 0u};
#if QLIN_WIDE_DIRECT_A
  // vmcnt(n) (expcnt and lgkmcnt left alone) before the barrier that ends
  // stage s: X of stage s + 1 was loaded during stage s - 1, followed by that
  // stage's W loads (B_LD) and, in stage s, the scale loads (W8: 2), the X
  // loads of stage s + 2 (A_LD) and the W loads (B_LD); loads complete in
  // issue order.  Six stages per round, so that every X and W buffer index
  // is a constant and the compiler keeps its waits partial.
  constexpr int kAfter = B_LD + (W8 ? 2 : 0) + A_LD + B_LD;
  static_assert(kAfter < 16, "vmcnt's low field");
  load_a_direct(0, 0);
  if (stages > 1) load_a_direct(1, 1);
  load_scales(0, csa);
  load(0, sl[0]);
  load(1, sl[1]);
  store(0, sl[0]);
  load(2, sl[0]);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // the prologue: everything in
  __syncthreads();
  if (stamp && tid == 0) stamp[kStampLoop] = __builtin_amdgcn_s_memrealtime();
  for (int g = 0; g < stages; g += 6) {
#pragma unroll
    for (int k = 0; k < 6; ++k) {
      const int st_ = g + k;  // this stage
      if (st_ >= stages) break;
      const bool next = st_ + 1 < stages;
      compute(k & 1, (k & 1) ? csb : csa, (k & 1) ? csa : csb, st_ + 1, next, (k + 1) & 1,
              &sl[(k + 1) & 1], true, st_ + 3, k % 3, st_ + 2 < stages, (k + 2) % 3);
      if (!next) break;
      // the next stage's X in and this stage's LDS accesses done, then a
      // bare barrier (a fence would also wait for the X loads of stage
      // st_ + 2, not needed before the barrier after the next)
      if (st_ + 2 < stages) {
        __builtin_amdgcn_s_waitcnt(0x0070 | kAfter);
      } else {
        __builtin_amdgcn_s_waitcnt(0x0070);
      }
      asm volatile("s_barrier" ::: "memory");
    }
  }
#else
  load_scales(0, csa);
  load(0, sl[0]);
  load(1, sl[1]);
  store(0, sl[0]);
  load(2, sl[0]);
  __syncthreads();
  if (stamp && tid == 0) stamp[kStampLoop] = __builtin_amdgcn_s_memrealtime();
  int g = 0;
  for (; g + 2 < stages; g += 2) {
    compute(0, csa, csb, g + 1, true, 1, &sl[1], true, g + 3, 0, false, 0);
    __syncthreads();
    compute(1, csb, csa, g + 2, true, 0, &sl[0], true, g + 4, 1, false, 0);
    __syncthreads();
  }
  {
    const bool more = g + 1 < stages;
    compute(0, csa, csb, g + 1, more, 1, &sl[1], false, 0, 0, false, 0);
    if (more) {
      __syncthreads();
      compute(1, csb, csa, g + 2, false, 0, &sl[0], false, 0, 1, false, 0);
    }
  }
#endif

  // Epilogue through LDS: the FP32 tile is staged row-major (element e of
  // tile (fm, fn) is row 8 (e / 4) + 4 h + e % 4, column r of that tile),
  // then each thread adds the bias to 8 consecutive columns of a row and
  // writes them as one 16-byte BF16 store.  Scattered 2-byte stores of the
  // accumulator layout cost several microseconds per tile.
  float* ep = reinterpret_cast<float*>(lds_raw);
  if (stamp && tid == 0) stamp[kStampEpilogue] = __builtin_amdgcn_s_memrealtime();
  __syncthreads();  // every wave is done with the stage buffers
#pragma unroll
  for (int fm = 0; fm < 2; ++fm)
#pragma unroll
    for (int fn = 0; fn < 2; ++fn)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = wm * 64 + fm * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        ep[row * kWideEpStride + wn * 64 + fn * 32 + r] = acc[fm][fn][e];
      }
  __syncthreads();
  constexpr int kChunksPerRow = BN / 8;
  constexpr int kChunks = BM * kChunksPerRow / NT;  // 8 per thread
  if (paired) {
    // 64 output columns: gate in tile columns 0-63, up in 64-127.  Each
    // thread takes 8 consecutive columns of 4 rows.  (Pair tiles are never
    // split over K.)
    constexpr int kPairPerRow = 64 / 8;
    constexpr int kPairChunks = BM * kPairPerRow / NT;  // 4 per thread
    const int col = (tid % kPairPerRow) * 8;
    const int n = n0 + col;
    float bg[8], bu[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const bool in = n + j < a.n;
      bg[j] = (a.bias && in) ? bf16_to_f32(gload(a.bias + n + j)) : 0.0f;
      bu[j] = (pair.bias2 && in) ? bf16_to_f32(gload(pair.bias2 + n + j)) : 0.0f;
    }
    const bool vec = (a.n % 8) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15u) == 0;
#pragma unroll
    for (int i = 0; i < kPairChunks; ++i) {
      const int row = (tid + NT * i) / kPairPerRow;
      const int m = m0 + row;
      if (m >= a.m || n >= a.n) continue;
      const int idx = row * (kWideEpStride / 4) + col / 4;
      const uint4 g0 = lds_raw[idx], g1 = lds_raw[idx + 1];
      const uint4 u0 = lds_raw[idx + 16], u1 = lds_raw[idx + 17];  // 64 columns on
      const float gf[8] = {__uint_as_float(g0.x), __uint_as_float(g0.y), __uint_as_float(g0.z),
                           __uint_as_float(g0.w), __uint_as_float(g1.x), __uint_as_float(g1.y),
                           __uint_as_float(g1.z), __uint_as_float(g1.w)};
      const float uf[8] = {__uint_as_float(u0.x), __uint_as_float(u0.y), __uint_as_float(u0.z),
                           __uint_as_float(u0.w), __uint_as_float(u1.x), __uint_as_float(u1.y),
                           __uint_as_float(u1.z), __uint_as_float(u1.w)};
      float o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        // the two GEMMs' BF16 outputs, then silu(g) * u
        const float g = bf16_to_f32(f32_to_bf16(gf[j] + bg[j]));
        const float u = bf16_to_f32(f32_to_bf16(uf[j] + bu[j]));
        o[j] = silu_mul_fast(g, u);
      }
      uint16_t* dst = a.y + static_cast<size_t>(m) * a.n + n;
      if (vec) {
        store_nt16(dst, u32x4{pack2_bf16(o[0], o[1]), pack2_bf16(o[2], o[3]),
                              pack2_bf16(o[4], o[5]), pack2_bf16(o[6], o[7])});
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (n + j < a.n) gstore(dst + j, f32_to_bf16(o[j]));
        }
      }
    }
    return;
  }
#if QLIN_WIDE_INKERNEL
  if (split.parts > 1) {
    if (split.xcd_local) {
      wide_split_handoff<true>(a, m0, n0, split, lds_raw, stamp);
    } else {
      wide_split_handoff<false>(a, m0, n0, split, lds_raw, stamp);
    }
    return;
  }
#endif
  if (split.parts > 1) {
    // One part of a tile split over K: its FP32 tile, row-major, for the
    // plan's reduction launch (the launch boundary orders these stores
    // before its loads) or, with split.help, for the workgroups of this
    // XCD (plain stores, kept in the XCD's L2; each thread waits for its
    // stores before wide_split_help counts the part).
    float* dst = split.partial + static_cast<size_t>(split.index) * (BM * BN);
    const int c8 = (tid % kChunksPerRow) * 8;
    if (split.help) {
#pragma unroll
      for (int i = 0; i < kChunks; ++i) {
        const int row = (tid + NT * i) / kChunksPerRow;
        const int idx = row * (kWideEpStride / 4) + c8 / 4;
        *(QLIN_GLOBAL u32x4*)(dst + row * BN + c8) = __builtin_bit_cast(u32x4, lds_raw[idx]);
        *(QLIN_GLOBAL u32x4*)(dst + row * BN + c8 + 4) =
            __builtin_bit_cast(u32x4, lds_raw[idx + 1]);
      }
      __builtin_amdgcn_s_waitcnt(0);
      return;
    }
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int row = (tid + NT * i) / kChunksPerRow;
      const int idx = row * (kWideEpStride / 4) + c8 / 4;
      store_nt16(dst + row * BN + c8, __builtin_bit_cast(u32x4, lds_raw[idx]));
      store_nt16(dst + row * BN + c8 + 4, __builtin_bit_cast(u32x4, lds_raw[idx + 1]));
    }
    return;
  }
  const int col = (tid % kChunksPerRow) * 8;  // the same for all of a thread's chunks
  const int n = n0 + col;
  // All LDS reads first (16-byte aligned: rows are kWideEpStride / 4 chunks
  // apart), then the stores, so no store waits behind a read.
  uint4 v[kChunks][2];
#pragma unroll
  for (int i = 0; i < kChunks; ++i) {
    const int row = (tid + NT * i) / kChunksPerRow;
    const int idx = row * (kWideEpStride / 4) + col / 4;
    v[i][0] = lds_raw[idx];
    v[i][1] = lds_raw[idx + 1];
  }
  float bias[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    bias[j] = (a.bias && n + j < a.n) ? bf16_to_f32(gload(a.bias + n + j)) : 0.0f;
  }
  const bool vec = (a.n % 8) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15u) == 0;
#pragma unroll
  for (int i = 0; i < kChunks; ++i) {
    const int m = m0 + (tid + NT * i) / kChunksPerRow;
    if (m >= a.m || n >= a.n) continue;
    float f[8];
    f[0] = __uint_as_float(v[i][0].x); f[1] = __uint_as_float(v[i][0].y);
    f[2] = __uint_as_float(v[i][0].z); f[3] = __uint_as_float(v[i][0].w);
    f[4] = __uint_as_float(v[i][1].x); f[5] = __uint_as_float(v[i][1].y);
    f[6] = __uint_as_float(v[i][1].z); f[7] = __uint_as_float(v[i][1].w);
    uint16_t* dst = a.y + static_cast<size_t>(m) * a.n + n;
    if (vec) {
      u32x4 o;
      o.x = pack2_bf16(f[0] + bias[0], f[1] + bias[1]);
      o.y = pack2_bf16(f[2] + bias[2], f[3] + bias[3]);
      o.z = pack2_bf16(f[4] + bias[4], f[5] + bias[5]);
      o.w = pack2_bf16(f[6] + bias[6], f[7] + bias[7]);
      store_nt16(dst, o);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (n + j < a.n) gstore(dst + j, f32_to_bf16(f[j] + bias[j]));
      }
    }
  }
}

template <bool W8>
__global__ __launch_bounds__(kWideThreads) void gemm_wide_kernel(GemmArgs a) {
  gemm_wide_tile<W8>(a, blockIdx.y * kWideRows, blockIdx.x * kWideCols);
}

// Row `row`, columns col .. col + 7 of a wide split tile summed over its
// `parts` FP32 parts (tile_partial: parts x 256 x 128 floats, row-major) in
// index order, plus the bias, written as BF16 to y[m, n .. n + 7] (y has N
// columns; m, n the row's and column's place in Y).  The one arithmetic of
// every wide split-K reduction, whichever workgroup runs it.
__device__ __forceinline__ void splitk_sum8(const float* tile_partial, int parts, int row,
                                            int col, const uint16_t* bias, uint16_t* y, int N,
                                            int m, int n) {
  const float* src = tile_partial + row * kWideCols + col;
  // parts in batches of four: a batch's loads are all issued before its adds
  constexpr int kBatch = 4;
  float f[8];
  for (int p0 = 0; p0 < parts; p0 += kBatch) {
    u32x4 v[kBatch][2];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      if (p0 + q < parts) {
        const float* sp = src + static_cast<size_t>(p0 + q) * (kWideRows * kWideCols);
        v[q][0] = *(const QLIN_GLOBAL u32x4*)(sp);
        v[q][1] = *(const QLIN_GLOBAL u32x4*)(sp + 4);
      }
    }
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      if (p0 + q < parts) {
        const float g[8] = {__uint_as_float(v[q][0].x), __uint_as_float(v[q][0].y),
                            __uint_as_float(v[q][0].z), __uint_as_float(v[q][0].w),
                            __uint_as_float(v[q][1].x), __uint_as_float(v[q][1].y),
                            __uint_as_float(v[q][1].z), __uint_as_float(v[q][1].w)};
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = (p0 + q) == 0 ? g[j] : f[j] + g[j];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (bias && n + j < N) f[j] += bf16_to_f32(gload(bias + n + j));
  }
  uint16_t* dst = y + static_cast<size_t>(m) * N + n;
  if ((N % 8) == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0) {
    store_nt16(dst, u32x4{pack2_bf16(f[0], f[1]), pack2_bf16(f[2], f[3]), pack2_bf16(f[4], f[5]),
                          pack2_bf16(f[6], f[7])});
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (n + j < N) gstore(dst + j, f32_to_bf16(f[j]));
    }
  }
}

// The in-launch reduction of a mapped launch's split tiles (map.help): the
// workgroups of XCD x (workgroup b runs on XCD b mod 8; the map keeps each
// split tile's parts on one XCD) sum the slices of that XCD's split tiles
// once their own units are done.  Slices (tile k of the XCD's list, slice s
// of kHelpSliceRows rows) are dealt round robin to the XCD's whole-tile
// workgroups by their rank in the map (to every workgroup of the XCD, by
// rank b / 8, if it has none), so no slice is claimed at run time.  Per tile (one 128-byte
// line ctr): a part adds 1 to ctr[0] once its FP32 tile is stored; a
// workgroup with a slice of the tile waits, a bounded number of polls, for
// every part and sums the slice (splitk_sum8: parts in index order, the
// reduction launch's arithmetic).  A workgroup that gives up waiting sets
// its slice's bit in ctr[3] and then adds kHelpAbandon to ctr[0]; if that
// add finds every part arrived it sums the slice after all.  The part whose
// add completes the count is the last: if the count it found holds an
// abandonment, it sums every slice marked in ctr[3].  The adds on ctr[0]
// are ordered, so each abandoned slice is summed by its workgroup or by the
// last part (some maybe by both, writing the same bytes), and nobody waits
// without bound.  Every workgroup of the XCD counts its departure from each
// of the XCD's tiles on ctr[2]; the last sets the tile's counters back to
// zero for the next launch.  The partial tiles are written and read with
// plain stores and loads inside the XCD's L2 (no reader has held those lines
// in its L1 this launch).
constexpr int kHelpSliceRows = 32;
constexpr int kHelpSlices = kWideRows / kHelpSliceRows;  // the bits of ctr[3]
constexpr int kHelpAbandon = 1 << 16;                      // > parts, x 256 fits an int

__device__ __forceinline__ int help_arrived(int* ctr) {
  return __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) % kHelpAbandon;
}

// Descriptor and tile of the launch's split tile T (numbered over the split
// descriptors in order); false if T is not one of them.
template <class DescAt>
__device__ __forceinline__ bool help_locate(DescAt desc_at, int count, int T, int* di, int* t) {
  int base = 0;
  for (int i = 0; i < count; ++i) {
    const GemmGroupDesc& e = desc_at(i);
    if (e.splits <= 1) continue;
    const int tiles = e.tiles_m * ((e.n + kWideCols - 1) / kWideCols);
    if (T < base + tiles) {
      *di = i;
      *t = T - base;
      return true;
    }
    base += tiles;
  }
  return false;
}

// Slice `slice` of tile t of d, 32 rows x 128 columns, 8 columns a thread.
__device__ __forceinline__ void help_sum_slice(const GemmGroupDesc& d, int t, int slice) {
  static_assert(kHelpSliceRows * (kWideCols / 8) == kWideThreads, "one row chunk a thread");
  const int tid = threadIdx.x;
  const int row = slice * kHelpSliceRows + tid / (kWideCols / 8);
  const int col = (tid % (kWideCols / 8)) * 8;
  const int m = (t % d.tiles_m) * kWideRows + row;
  const int n = (t / d.tiles_m) * kWideCols + col;
  if (m < d.m && n < d.n) {
    splitk_sum8(d.partial + static_cast<size_t>(t) * d.splits * (kWideRows * kWideCols),
                d.splits, row, col, d.bias, d.y, d.n, m, n);
  }
}

template <class DescAt>
__device__ __forceinline__ void wide_split_help(DescAt desc_at, int count, const WideBlockMap& map,
                                                int own, unsigned long long* stamp = nullptr) {
  __shared__ int word;
  const int tid = threadIdx.x;
  const int x = static_cast<int>(blockIdx.x) % kXcds;
  const int members = (static_cast<int>(gridDim.x) - x + kXcds - 1) / kXcds;
  const int helpers = map.help_members[x];
  const int rank = helpers > 0 ? map.help_rank[blockIdx.x] : static_cast<int>(blockIdx.x) / kXcds;
  const int dealt = helpers > 0 ? helpers : members;
  int tiles = 0;
  while (tiles < kHelpTiles && map.help_tiles[x][tiles] != 0xFF) ++tiles;
  __syncthreads();  // a part: every thread's partial stores are done
  int own_di = 0, own_t = 0;
  if (own >= 0 && help_locate(desc_at, count, own, &own_di, &own_t)) {
    const GemmGroupDesc& d = desc_at(own_di);
    int* ctr = d.counters + static_cast<size_t>(own_t) * kHelpCounterInts;
    if (tid == 0) {
      const int before = __hip_atomic_fetch_add(&ctr[0], 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
      // last part, after an abandonment: the abandoned slices (0: none)
      word = before % kHelpAbandon == d.splits - 1 && before >= kHelpAbandon
                 ? __hip_atomic_load(&ctr[3], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                 : 0;
    }
    __syncthreads();
    const int abandoned = word;
    for (int slice = 0; slice < kHelpSlices; ++slice) {
      if (abandoned & (1 << slice)) help_sum_slice(d, own_t, slice);
    }
    __syncthreads();  // `word` is free again
  }
  // this workgroup's slices
  bool first = true;
  for (int j = rank; rank != 0xFF && j < tiles * kHelpSlices; j += dealt) {
    int di, t;
    if (!help_locate(desc_at, count, map.help_tiles[x][j / kHelpSlices], &di, &t)) continue;
    const GemmGroupDesc& d = desc_at(di);
    int* ctr = d.counters + static_cast<size_t>(t) * kHelpCounterInts;
    const int slice = j % kHelpSlices;
    if (tid == 0) {
      bool arrived = false;
      for (int poll = 0; poll < kWideArrivePolls && !arrived; ++poll) {
        arrived = help_arrived(&ctr[0]) >= d.splits;
        if (!arrived) __builtin_amdgcn_s_sleep(2);
      }
      if (!arrived) {  // give the slice to the last part, unless it has come
        __hip_atomic_fetch_or(&ctr[3], 1 << slice, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);  // the bit is set before the add is counted
        arrived = __hip_atomic_fetch_add(&ctr[0], kHelpAbandon, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT) % kHelpAbandon >= d.splits;
      }
      word = arrived;
    }
    __syncthreads();
    const bool arrived = word != 0;
    if (stamp && first && tid == 0) stamp[kStampArrived] = __builtin_amdgcn_s_memrealtime();
    first = false;
    if (arrived) help_sum_slice(d, t, slice);
    __syncthreads();  // every thread has read `word`
  }
  if (stamp && tid == 0) stamp[kStampReduced] = __builtin_amdgcn_s_memrealtime();
  // departures (lanes 0 .. tiles - 1 of wave 0, one tile each, all at once):
  // the last workgroup of the XCD to leave a tile resets its counters
  if (tid < tiles) {
    int di, t;
    if (help_locate(desc_at, count, map.help_tiles[x][tid], &di, &t)) {
      int* ctr = desc_at(di).counters + static_cast<size_t>(t) * kHelpCounterInts;
      if (__hip_atomic_fetch_add(&ctr[2], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
          members - 1) {
        __hip_atomic_store(&ctr[0], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&ctr[2], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&ctr[3], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// The launch-wide number of split tile `u` of descriptor `lo` (split tiles
// numbered over the launch's split descriptors in order, as
// map_wide_group_to_xcds numbers them), or -1 for a whole or pair tile.
template <class DescAt>
__device__ __forceinline__ int own_split_tile(DescAt desc_at, int lo, int u) {
  const GemmGroupDesc& d = desc_at(lo);
  if (d.splits <= 1) return -1;
  int base = 0;
  for (int i = 0; i < lo; ++i) {
    const GemmGroupDesc& e = desc_at(i);
    if (e.splits > 1) base += e.tiles_m * ((e.n + kWideCols - 1) / kWideCols);
  }
  return base + u / d.splits;
}

// Grouped form of gemm_wide_kernel (same block -> unit mapping as
// gemm_grouped_kernel: part u % splits of tile u / splits, M tiles fastest).
template <bool W8>
__device__ __forceinline__ void gemm_wide_unit(const GemmGroupDesc& d, int u, bool xcd_local,
                                               unsigned long long* stamp = nullptr,
                                               bool help = false) {
  const int tile = u / d.splits;
  if (d.w2) {
    // A gate|up pair: d.n counts both halves; each tile 64 columns of each.
    const GemmArgs a{d.w, d.s, d.bias, d.x, d.y, d.m, d.n / 2, d.k};
    gemm_wide_tile<W8>(a, (tile % d.tiles_m) * kWideRows, (tile / d.tiles_m) * (kWideCols / 2),
                       SplitK{}, WidePair{d.w2, d.s2, d.bias2}, stamp);
    return;
  }
  const GemmArgs a{d.w, d.s, d.bias, d.x, d.y, d.m, d.n, d.k};
  SplitK sp;
  if (d.splits > 1) {
    const int groups = d.k / kStageK;
    sp.parts = d.splits;
    sp.index = u % d.splits;
    sp.begin = sp.index * d.split_stages;
    sp.count = min(d.split_stages, groups - sp.begin);
    sp.partial = d.partial + static_cast<size_t>(tile) * d.splits * (kWideRows * kWideCols);
    sp.counter = d.counters ? d.counters + static_cast<size_t>(tile) * kWideSplitCounterInts : nullptr;
    sp.xcd_local = QLIN_HANDOFF_L2 && xcd_local;
    sp.help = help;
  }
  gemm_wide_tile<W8>(a, (tile % d.tiles_m) * kWideRows, (tile / d.tiles_m) * kWideCols, sp,
                     WidePair{}, stamp);
}

template <bool W8>
__global__ __launch_bounds__(kWideThreads) void gemm_wide_grouped_kernel(
    const GemmGroupDesc* __restrict__ descs, int count, WideBlockMap map) {
  const int b = map.mapped ? map.logical[blockIdx.x] : blockIdx.x;
  int lo = 0, hi = count - 1;
  while (lo < hi) {  // last descriptor whose block_begin <= b
    const int mid = (lo + hi + 1) >> 1;
    if (descs[mid].block_begin <= b) lo = mid; else hi = mid - 1;
  }
  gemm_wide_unit<W8>(descs[lo], b - descs[lo].block_begin, map.mapped != 0, nullptr,
                     QLIN_WIDE_HELP && map.help);
  if (QLIN_WIDE_HELP && map.help) {
    auto at = [&](int i) -> const GemmGroupDesc& { return descs[i]; };
    wide_split_help(at, count, map, own_split_tile(at, lo, b - descs[lo].block_begin));
  }
}

// gemm_wide_grouped_kernel with a timeline: workgroup w writes the
// WideStamp slots stamps[w * kStampSlots ..] (a measurement launch; the
// stores and barrier at the end are its only extra work).  t0 and c0 are
// the clocks read at the kernel's first instruction.
template <bool W8, class DescAt>
__device__ __forceinline__ void wide_timeline_unit(DescAt desc_at, int count, int lo, int b,
                                                   const WideBlockMap& map,
                                                   unsigned long long t0, unsigned long long c0,
                                                   unsigned long long* __restrict__ stamps) {
  const GemmGroupDesc& d = desc_at(lo);
  const bool xcd_local = map.mapped != 0;
  unsigned long long* stamp = stamps + static_cast<size_t>(blockIdx.x) * kStampSlots;
  const int u = b - d.block_begin;
  const int groups = d.k / kStageK;
  const int stages =
      d.splits > 1 ? min(d.split_stages, groups - (u % d.splits) * d.split_stages) : groups;
  const int kind = d.w2 ? 2 : (d.splits > 1 ? 1 : 0);
  if (threadIdx.x == 0) {
    unsigned xcc, hwid;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hwid));
    stamp[kStampEntry] = t0;
    stamp[kStampXcc] = xcc;
    stamp[kStampHwId] = hwid;
    stamp[kStampUnit] = static_cast<unsigned long long>(b) |
                        (static_cast<unsigned long long>(stages) << 16) |
                        (static_cast<unsigned long long>(kind) << 24);
  }
  gemm_wide_unit<W8>(d, u, xcd_local, stamp, QLIN_WIDE_HELP && map.help);
  if (QLIN_WIDE_HELP && map.help) {
    if (threadIdx.x == 0) stamp[kStampHelp] = __builtin_amdgcn_s_memrealtime();
    wide_split_help(desc_at, count, map, own_split_tile(desc_at, lo, u), stamp);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    stamp[kStampEnd] = __builtin_amdgcn_s_memrealtime();
    stamp[kStampCycles] = __builtin_amdgcn_s_memtime() - c0;
  }
}

template <bool W8>
__global__ __launch_bounds__(kWideThreads) void gemm_wide_grouped_timeline_kernel(
    const GemmGroupDesc* __restrict__ descs, int count, WideBlockMap map,
    unsigned long long* __restrict__ stamps) {
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  const int b = map.mapped ? map.logical[blockIdx.x] : blockIdx.x;
  int lo = 0, hi = count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (descs[mid].block_begin <= b) lo = mid; else hi = mid - 1;
  }
  auto at = [&](int i) -> const GemmGroupDesc& { return descs[i]; };
  wide_timeline_unit<W8>(at, count, lo, b, map, t0, c0, stamps);
}

template <bool W8>
__global__ __launch_bounds__(kWideThreads) void gemm_wide_inline_timeline_kernel(
    GemmGroupArgs g, WideBlockMap map, unsigned long long* __restrict__ stamps) {
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  const int b = map.mapped ? map.logical[blockIdx.x] : blockIdx.x;
  int lo = 0;
#pragma unroll
  for (int i = 1; i < kInlineGroupMax; ++i) {
    if (i < g.count && g.d[i].block_begin <= b) lo = i;
  }
  auto at = [&](int i) -> const GemmGroupDesc& { return g.d[i]; };
  wide_timeline_unit<W8>(at, g.count, lo, b, map, t0, c0, stamps);
}

// The same with the descriptors in the kernel arguments.
template <bool W8>
__global__ __launch_bounds__(kWideThreads) void gemm_wide_inline_kernel(GemmGroupArgs g,
                                                                       WideBlockMap map) {
  const int b = map.mapped ? map.logical[blockIdx.x] : blockIdx.x;
  int lo = 0;
#pragma unroll
  for (int i = 1; i < kInlineGroupMax; ++i) {
    if (i < g.count && g.d[i].block_begin <= b) lo = i;
  }
  gemm_wide_unit<W8>(g.d[lo], b - g.d[lo].block_begin, map.mapped != 0, nullptr,
                     QLIN_WIDE_HELP && map.help);
  if (QLIN_WIDE_HELP && map.help) {
    auto at = [&](int i) -> const GemmGroupDesc& { return g.d[i]; };
    wide_split_help(at, g.count, map, own_split_tile(at, lo, b - g.d[lo].block_begin));
  }
}

// Split-K reduction, the second launch of a wide-tile plan: each block sums
// 16 rows of one split tile over its parts in index order (the result does
// not depend on which part finished first), adds the bias and writes BF16;
// each thread 8 consecutive columns of one row.
__device__ __forceinline__ void splitk_reduce_block(const SplitReduceDesc& d, int b) {
  constexpr int kBlocksPerTile = kWideRows / kSplitReduceRows;
  const int u = b - d.block_begin;
  const int tile = u / kBlocksPerTile;
  const int row = (u % kBlocksPerTile) * kSplitReduceRows + threadIdx.x / 16;
  const int col = (threadIdx.x % 16) * 8;
  const int m = (tile % d.tiles_m) * kWideRows + row;
  const int n = (tile / d.tiles_m) * kWideCols + col;
  if (m >= d.m || n >= d.n) return;
  splitk_sum8(d.partial + static_cast<size_t>(tile) * d.parts * (kWideRows * kWideCols), d.parts,
              row, col, d.bias, d.y, d.n, m, n);
}

// The logical reduction block of workgroup w (-1: none).  Mapped: XCD w % 8,
// row block k % 16 of the split tile in slot k / 16 of that XCD (k = w / 8).
__device__ __forceinline__ int reduce_block(const ReduceBlockMap& map, int w) {
  if (map.slots == 0) return w;
  constexpr int kBlocksPerTile = kWideRows / kSplitReduceRows;
  const int k = w / kXcds;
  const int t = map.tile[w % kXcds][k / kBlocksPerTile];
  return t == 0xFF ? -1 : t * kBlocksPerTile + k % kBlocksPerTile;
}

__global__ __launch_bounds__(256) void splitk_reduce_kernel(
    const SplitReduceDesc* __restrict__ descs, int count, ReduceBlockMap map) {
  const int b = reduce_block(map, blockIdx.x);
  if (b < 0) return;
  int lo = 0, hi = count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (descs[mid].block_begin <= b) lo = mid; else hi = mid - 1;
  }
  splitk_reduce_block(descs[lo], b);
}

__global__ __launch_bounds__(256) void splitk_reduce_inline_kernel(SplitReduceArgs r,
                                                                   ReduceBlockMap map) {
  const int b = reduce_block(map, blockIdx.x);
  if (b < 0) return;
  int lo = 0;
#pragma unroll
  for (int i = 1; i < kInlineGroupMax; ++i) {
    if (i < r.count && r.d[i].block_begin <= b) lo = i;
  }
  splitk_reduce_block(r.d[lo], b);
}

// Grid: x = N tiles, y = M tiles.
template <int BM, int BN, int WAVES_M, bool W8>
__global__ __launch_bounds__(kThreads) QLIN_GEMM_WAVES_ATTR void gemm_mfma_kernel(GemmArgs a) {
  gemm_tile<BM, BN, WAVES_M, W8, kPrefetch>(a, blockIdx.y * BM, blockIdx.x * BN);
}

// Many GEMMs in one launch.  Block b belongs to the descriptor d with
// block_begin[d] <= b < block_begin[d + 1] (descriptors sorted by
// block_begin); its unit u = b - block_begin[d] is part u % splits of
// output tile u / splits, M tiles fastest (consecutive tiles share one
// weight tile).
template <int BM, int BN, int WAVES_M, bool W8>
__device__ __forceinline__ void gemm_grouped_unit(const GemmGroupDesc& d, int u) {
  const int tile = u / d.splits;
  const GemmArgs a{d.w, d.s, d.bias, d.x, d.y, d.m, d.n, d.k};
  SplitK sp;
  if (d.splits > 1) {
    const int groups = d.k / kStageK;
    sp.parts = d.splits;
    sp.index = u % d.splits;
    sp.begin = sp.index * d.split_stages;
    sp.count = min(d.split_stages, groups - sp.begin);
    sp.partial = d.partial + static_cast<size_t>(tile) * d.splits * (BM * BN);
    sp.counter = d.counters + tile;
  }
  gemm_tile<BM, BN, WAVES_M, W8, kPrefetch>(a, (tile % d.tiles_m) * BM, (tile / d.tiles_m) * BN,
                                            sp, &d);
}

template <int BM, int BN, int WAVES_M, bool W8>
__global__ __launch_bounds__(kThreads) QLIN_GEMM_WAVES_ATTR void gemm_grouped_kernel(
    const GemmGroupDesc* __restrict__ descs, int count) {
  const int b = blockIdx.x;
  int lo = 0, hi = count - 1;
  while (lo < hi) {  // last descriptor whose block_begin <= b
    const int mid = (lo + hi + 1) >> 1;
    if (descs[mid].block_begin <= b) lo = mid; else hi = mid - 1;
  }
  gemm_grouped_unit<BM, BN, WAVES_M, W8>(descs[lo], b - descs[lo].block_begin);
}

template <int BM, int BN, int WAVES_M, bool W8>
__global__ __launch_bounds__(kThreads) QLIN_GEMM_WAVES_ATTR void gemm_grouped_inline_kernel(
    GemmGroupArgs g) {
  const int b = blockIdx.x;
  int lo = 0;
#pragma unroll
  for (int i = 1; i < kInlineGroupMax; ++i) {
    if (i < g.count && g.d[i].block_begin <= b) lo = i;
  }
  gemm_grouped_unit<BM, BN, WAVES_M, W8>(g.d[lo], b - g.d[lo].block_begin);
}

template <int BM, int BN, int WAVES_M, bool W8>
void launch_tile(const GemmArgs& a, hipStream_t stream) {
  const dim3 grid((a.n + BN - 1) / BN, (a.m + BM - 1) / BM);
  hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, WAVES_M, W8>), grid, dim3(kThreads), 0, stream,
                     a);
}

template <bool W8>
void launch_config(int config, const GemmArgs& a, hipStream_t stream) {
  switch (config) {
    case kGemmTile128x128: launch_tile<128, 128, 2, W8>(a, stream); break;
    case kGemmTile128x64: launch_tile<128, 64, 2, W8>(a, stream); break;
    case kGemmTile64x128: launch_tile<64, 128, 2, W8>(a, stream); break;
    case kGemmTile64x64: launch_tile<64, 64, 2, W8>(a, stream); break;
    case kGemmTile32x128: launch_tile<32, 128, 1, W8>(a, stream); break;
    case kGemmTile256x128: {
      const dim3 grid((a.n + kWideCols - 1) / kWideCols, (a.m + kWideRows - 1) / kWideRows);
      hipLaunchKernelGGL((gemm_wide_kernel<W8>), grid, dim3(kWideThreads), 0, stream, a);
      break;
    }
    default: launch_tile<64, 64, 2, W8>(a, stream); break;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ------------------------------------------------------------------------
// Skinny GEMM: Y[m, n] for a few tokens (up to kSkinnyMaxTokens), the
// weights streamed once per 32 tokens.
//
// With a few tokens a GEMM is bound by reading its weights (15.4 MB of int8
// per Qwen2.5-0.5B layer), not by MFMA: staging 64 x 64 tiles through LDS
// leaves a few dozen workgroups walking 14 dependent stages each.  Here a
// workgroup owns 32 weight rows of one Linear (the MFMA's 32 columns) and
// one tile of 32 tokens (its 32 rows); its KW waves split K, each issuing
// all the weight and activation loads of a round of up to four 64-column
// groups at once, and the waves' accumulators are summed in LDS in wave
// order.  The loads are coalesced (a group's 64-column rows across
// consecutive lanes) and each wave permutes them into MFMA fragments
// through its own slice of LDS, which needs no workgroup barrier.
//
// Lane (r, h) feeds MFMA k-step ks of group g with chunk 4 h + ks of the
// group (K 64 g + 32 h + 8 ks .. + 7), for the A fragment of token r and
// the B fragment of weight row n0 + r: the fragments the 64 x 64 tile
// kernel reads from LDS, so a group's MFMA partial is the same, and its
// W8A16 scale (row n0 + r, group g) is one value per lane.  Accumulator
// element e is token m0 + 8 (e / 4) + 4 h + e % 4 of row n0 + r.  Buffer
// loads whose offset is past the operand (tokens >= m, rows >= n) read
// zeros.
//
// PAIR: the workgroup computes gate (w, s, bias) and up (w2, s2, bias2)
// rows n0 .. n0 + 31 and writes bf16(silu(bf16(gate)) * bf16(up)).
// A GEMM split over K (d.parts > 1) runs `parts` workgroups per row block
// and token tile; their wave 0s hand off through d.partial as the 64 x 64
// tiles' split-K does (device-coherent stores, an agent-scope arrival
// count, the last one summing the parts in index order and resetting the
// count), with no workgroup barrier: only wave 0 takes part.
template <bool W8, bool PAIR, int KW>
__global__ __launch_bounds__(kWave * KW) void gemm_skinny_kernel(SkinnyArgs a) {
  constexpr int kRound = 4;  // groups per wave per round of loads
  const int b = blockIdx.x;
  SkinnyDesc d = a.d[0];  // the last descriptor whose block_begin <= b
#pragma unroll
  for (int i = 1; i < kSkinnyMaxDescs; ++i) {
    if (i < a.count && a.d[i].block_begin <= b) d = a.d[i];
  }
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int r = lane & 31, h = lane >> 5;
  // workgroup = (row block, token tile of 32, K part), part fastest
  const int tiles_t = (a.m + 31) / 32;
  const int local = b - d.block_begin;
  const int part = local % d.parts, tt = local / d.parts % tiles_t;
  const int rb = local / d.parts / tiles_t;
  const int n0 = rb * 32, m0 = tt * 32;
  const int tile = rb * tiles_t + tt;  // split-K counter and partials
  const int groups = d.k / kStageK;
  // this part's groups, then this wave's share of them
  const int per_part = (groups + d.parts - 1) / d.parts;
  const int p_begin = min(groups, part * per_part), p_end = min(groups, p_begin + per_part);
  const int per = (p_end - p_begin + KW - 1) / KW;
  const int g_begin = min(p_end, p_begin + wave * per), g_end = min(p_end, g_begin + per);
  const uint32_t wbytes = W8 ? 1u : 2u;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(d.x + static_cast<size_t>(m0) * d.k,
                                              static_cast<uint32_t>(a.m - m0) * d.k * 2u);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(d.w, static_cast<uint32_t>(d.n) * d.k * wbytes);
  const __amdgpu_buffer_rsrc_t wr2 =
      make_rsrc(PAIR ? d.w2 : d.w, static_cast<uint32_t>(d.n) * d.k * wbytes);
  // Lane offsets of group 0; group g adds 64 g columns (a scalar offset).
  // X goes through this wave's LDS slice: load i of a group brings tokens
  // 8 i .. 8 i + 7, lane l chunk l % 8 of token 8 i + l / 8 (eight lanes per
  // 128-byte row: one cache line per eight lanes, where loading fragments
  // directly touches a line per lane), and the fragments are read back from
  // LDS, one group at a time through one 4 KB slot per wave.  The wave's own
  // LDS accesses execute in order: no barrier.
  __shared__ uint4 lds_x[KW][32 * kRowChunks];
  const uint32_t xoff =
      (static_cast<uint32_t>(lane >> 3) * d.k + 8u * (lane & 7)) * 2u;  // + 8 i rows
  const uint32_t xrow8 = 8u * d.k * 2u;
  // W likewise: int8 rows of a group are 64 bytes, four lanes per row,
  // loads of 16 rows (pieces swizzled in LDS against bank conflicts); BF16
  // rows as X's, loads of 8 rows.
  constexpr int kWSlots = W8 ? 32 * 4 : 32 * kRowChunks;
  __shared__ uint4 lds_w[KW][PAIR ? 2 : 1][kWSlots];
  const uint32_t woff =
      W8 ? static_cast<uint32_t>(n0 + (lane >> 2)) * d.k + 16u * (lane & 3)
         : (static_cast<uint32_t>(n0 + (lane >> 3)) * d.k + 8u * (lane & 7)) * 2u;
  const uint32_t wrows = (W8 ? 16u : 8u) * d.k * wbytes;  // between a group's loads
  auto w_slot = [](int row, int piece) {
    return W8 ? row * 4 + (piece ^ ((row >> 2) & 3)) : lds_slot(row, piece);
  };
  const int srow = min(n0 + r, d.n - 1);  // scales: clamped row, its value unused past N
  const uint16_t* s1 = W8 ? d.s + static_cast<size_t>(srow) * groups : nullptr;
  const uint16_t* s2 = W8 && PAIR ? d.s2 + static_cast<size_t>(srow) * groups : nullptr;

  f32x16_t acc = {}, acc2 = {};
  for (int g0 = g_begin; g0 < g_end; g0 += kRound) {
    // One round: the loads of up to kRound groups, issued together (groups
    // past g_end re-read the round's first group and are not used).
    uint4 xa[kRound][4], wq[kRound][W8 ? 2 : 4], wq2[kRound][PAIR ? (W8 ? 2 : 4) : 1];
    uint32_t sc[kRound], sc2[kRound];
#pragma unroll
    for (int j = 0; j < kRound; ++j) {
      const uint32_t g = static_cast<uint32_t>(g0 + j < g_end ? g0 + j : g0);
#pragma unroll
      for (int i = 0; i < (W8 ? 2 : 4); ++i) {
        wq[j][i] = buffer_load16(wr, woff + wrows * i, g * kStageK * wbytes);
        if (PAIR) wq2[j][i] = buffer_load16(wr2, woff + wrows * i, g * kStageK * wbytes);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) xa[j][i] = buffer_load16(xr, xoff + xrow8 * i, g * kStageK * 2u);
      if (W8) {
        sc[j] = gload(s1 + g);
        if (PAIR) sc2[j] = gload(s2 + g);
      }
    }
#pragma unroll
    for (int j = 0; j < kRound; ++j) {
      if (g0 + j >= g_end) break;
      // X: the coalesced pieces into LDS, the fragments back out
#pragma unroll
      for (int i = 0; i < 4; ++i) lds_x[wave][lds_slot(8 * i + (lane >> 3), lane & 7)] = xa[j][i];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) xa[j][ks] = lds_x[wave][lds_slot(r, 4 * h + ks)];
      // W: the same; a lane then holds int8 pieces 2 h, 2 h + 1 (chunks
      // 4 h .. 4 h + 3) or BF16 chunks 4 h .. 4 h + 3 of row n0 + r
      constexpr int kRowsPerLoad = W8 ? 16 : 8, kLanesPerRow = W8 ? 4 : 8;
#pragma unroll
      for (int i = 0; i < (W8 ? 2 : 4); ++i) {
        const int slot = w_slot(kRowsPerLoad * i + lane / kLanesPerRow, lane % kLanesPerRow);
        lds_w[wave][0][slot] = wq[j][i];
        if (PAIR) lds_w[wave][PAIR ? 1 : 0][slot] = wq2[PAIR ? j : 0][PAIR ? i : 0];
      }
#pragma unroll
      for (int i = 0; i < (W8 ? 2 : 4); ++i) {
        const int slot = w_slot(r, (W8 ? 2 : 4) * h + i);
        wq[j][i] = lds_w[wave][0][slot];
        if (PAIR) wq2[PAIR ? j : 0][PAIR ? i : 0] = lds_w[wave][PAIR ? 1 : 0][slot];
      }
      bf16x8_t fb[4], fb2[4];
      if (W8) {
        uint4 lo, hi;
        i8x16_to_bf16(wq[j][0], lo, hi);
        fb[0] = as_bf16x8(lo);
        fb[1] = as_bf16x8(hi);
        i8x16_to_bf16(wq[j][1], lo, hi);
        fb[2] = as_bf16x8(lo);
        fb[3] = as_bf16x8(hi);
        if (PAIR) {
          i8x16_to_bf16(wq2[j][0], lo, hi);
          fb2[0] = as_bf16x8(lo);
          fb2[1] = as_bf16x8(hi);
          i8x16_to_bf16(wq2[j][1], lo, hi);
          fb2[2] = as_bf16x8(lo);
          fb2[3] = as_bf16x8(hi);
        }
      } else {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          fb[ks] = as_bf16x8(wq[j][ks]);
          if (PAIR) fb2[ks] = as_bf16x8(wq2[PAIR ? j : 0][PAIR ? ks : 0]);
        }
      }
      if (W8) {
        const f32x16_t zero = {};
        f32x16_t part = zero, part2 = zero;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          part = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(xa[j][ks]), fb[ks],
                                                         ks == 0 ? zero : part, 0, 0, 0);
          if (PAIR) {
            part2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(xa[j][ks]), fb2[ks],
                                                            ks == 0 ? zero : part2, 0, 0, 0);
          }
        }
        const float s = bf16_to_f32(sc[j]);
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = fmaf(part[e], s, acc[e]);
        if (PAIR) {
          const float t = bf16_to_f32(sc2[j]);
#pragma unroll
          for (int e = 0; e < 16; ++e) acc2[e] = fmaf(part2[e], t, acc2[e]);
        }
      } else {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(xa[j][ks]), fb[ks], acc, 0,
                                                        0, 0);
          if (PAIR) {
            acc2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(xa[j][ks]), fb2[ks], acc2,
                                                           0, 0, 0);
          }
        }
      }
    }
  }

  // The waves' accumulators, summed in wave order by wave 0.
  if (KW > 1) {
    __shared__ f32x4_t red[KW > 1 ? KW : 1][PAIR ? 2 : 1][4][kWave];
    if (wave > 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        red[wave][0][q][lane] = f32x4_t{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
        if (PAIR) {
          red[wave][PAIR ? 1 : 0][q][lane] =
              f32x4_t{acc2[4 * q], acc2[4 * q + 1], acc2[4 * q + 2], acc2[4 * q + 3]};
        }
      }
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 1; w < KW; ++w) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4_t v = red[w][0][q][lane];
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[4 * q + t] += v[t];
        if (PAIR) {
          const f32x4_t v2 = red[w][PAIR ? 1 : 0][q][lane];
#pragma unroll
          for (int t = 0; t < 4; ++t) acc2[4 * q + t] += v2[t];
        }
      }
    }
  }

  if (!PAIR && d.parts > 1) {
    // Split-K hand-off (wave 0 only).  Lane l's 16 values are 4 16-byte
    // vectors at [(q * 64 + l) * 4] of the part's 1024 floats.
    const __amdgpu_buffer_rsrc_t pr =
        make_rsrc(d.partial + static_cast<size_t>(tile) * d.parts * 1024,
                  static_cast<uint32_t>(d.parts) * 4096u);
    const uint32_t mine = static_cast<uint32_t>(part) * 4096u;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4_t v = {acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), pr,
                                             mine + (q * kWave + lane) * 16u, 0, kCoherent);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this lane's part is stored
    int arrived = 0;
    if (lane == 0) {
      arrived = __hip_atomic_fetch_add(d.counters + tile, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
    }
    if (__builtin_amdgcn_readfirstlane(arrived) != d.parts - 1) return;
    f32x16_t sum;
    for (int p = 0; p < d.parts; ++p) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4_t v;
        if (p == part) {
          v = f32x4_t{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
        } else {
          v = __builtin_bit_cast(
              f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                           pr, static_cast<uint32_t>(p) * 4096u + (q * kWave + lane) * 16u, 0,
                           kCoherent));
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) sum[4 * q + c] = p == 0 ? v[c] : sum[4 * q + c] + v[c];
      }
    }
    acc = sum;
    if (lane == 0) {  // ready for the next launch
      __hip_atomic_store(d.counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  const int n = n0 + r;
  if (n >= d.n) return;
  const float bias = d.bias ? bf16_to_f32(gload(d.bias + n)) : 0.0f;
  const float bias2 = PAIR && d.bias2 ? bf16_to_f32(gload(d.bias2 + n)) : 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int m = m0 + 8 * (e >> 2) + 4 * h + (e & 3);
    if (m >= a.m) continue;
    float v;
    if (PAIR) {
      // silu(g) * u on the two BF16 GEMM outputs
      const float gv = bf16_to_f32(f32_to_bf16(acc[e] + bias));
      const float uv = bf16_to_f32(f32_to_bf16(acc2[e] + bias2));
      v = silu_mul_fast(gv, uv);
    } else {
      v = acc[e] + bias;
    }
    gstore(d.y + static_cast<size_t>(m) * d.n + n, f32_to_bf16(v));
  }
}

template <bool W8, bool PAIR>
void launch_skinny_kw(const SkinnyArgs& a, int blocks, int kw, hipStream_t stream) {
  switch (kw) {
    case 1:
      hipLaunchKernelGGL((gemm_skinny_kernel<W8, PAIR, 1>), dim3(blocks), dim3(kWave), 0, stream, a);
      break;
    case 2:
      hipLaunchKernelGGL((gemm_skinny_kernel<W8, PAIR, 2>), dim3(blocks), dim3(2 * kWave), 0,
                         stream, a);
      break;
    case 4:
      hipLaunchKernelGGL((gemm_skinny_kernel<W8, PAIR, 4>), dim3(blocks), dim3(4 * kWave), 0,
                         stream, a);
      break;
    default:
      // (a pair holds twice the registers: at most 4 waves, 256 each;
      // layout_skinny never asks a pair for more)
      if constexpr (PAIR) {
        hipLaunchKernelGGL((gemm_skinny_kernel<W8, PAIR, 4>), dim3(blocks), dim3(4 * kWave), 0,
                           stream, a);
      } else {
        hipLaunchKernelGGL((gemm_skinny_kernel<W8, PAIR, 8>), dim3(blocks), dim3(8 * kWave), 0,
                           stream, a);
      }
      break;
  }
}

}  // namespace

bool gemm_mfma_supported(const void* w, const uint16_t* x, int m, int n, int k) {
  // Buffer loads address each operand with a 32-bit byte offset.
  const long long limit = 0x7FFFFFFFll;
  return k >= kStageK && k % kStageK == 0 && aligned16(w) && aligned16(x) &&
         2ll * m * k < limit && 2ll * n * k < limit;
}

bool gemm_skinny_supported(const void* w, const uint16_t* x, int m, int n, int k) {
  return m >= 1 && m <= kSkinnyMaxTokens && n >= 1 && gemm_mfma_supported(w, x, m, n, k);
}

bool gemm_skinny_preferred(bool w8, int m, int n, int k) {
  // Single calls on MI355X, us (skinny / 64 x 64 tile), W8A16: M = 32 q
  // 5.1 / 7.1, gate 5.6 / 7.1, down 11.7 / 29.1; M = 64 gate 6.9 / 7.1;
  // M = 128 q 5.2 / 7.1, gate 8.5 / 8.1, down 12.5 / 30.0.  BF16: M = 64 q
  // 5.0 / 5.4, gate 7.2 / 6.5; M = 128 q 5.9 / 5.5, down 12.4 / 22.8.
  if (m <= 32 || (w8 && m <= 64)) return true;
  if (m > kSkinnyMaxTokens || n > 1024) return false;
  return w8 || m <= 64 || k >= 2048;
}

int layout_skinny(SkinnyArgs& a, bool split) {
  // About four groups of 64 per wave: one round of loads.  Without a split,
  // up to 8 waves per workgroup (two per SIMD keep 256 registers per wave;
  // 4 for a pair, whose rounds hold both weights).  With it, 4 waves and a
  // GEMM longer than 16 groups in parts of at most 16: a lone row block per
  // CU cannot pull its weights and activations fast enough (down_proj at 32
  // tokens: 28 workgroups of 8 waves took 16.9 us).
  const bool pair = a.d[0].w2 != nullptr;
  int groups = 0;
  for (int i = 0; i < a.count; ++i) groups = std::max(groups, a.d[i].k / kStageK);
  int kw = 1;
  if (split && !pair) {
    kw = 4;
  } else {
    while (kw < (pair ? 4 : 8) && kw * 4 < groups) kw *= 2;
  }
  a.waves = kw;
  int blocks = 0;
  for (int i = 0; i < a.count; ++i) {
    SkinnyDesc& d = a.d[i];
    const int g = d.k / kStageK;
    d.parts = split && !pair && g > 16 ? (g + 15) / 16 : 1;
    d.partial = nullptr;
    d.counters = nullptr;
    d.block_begin = blocks;
    blocks += (d.n + 31) / 32 * ((a.m + 31) / 32) * d.parts;
  }
  return blocks;
}

void skinny_scratch(const SkinnyArgs& a, size_t* partial_floats, size_t* counters) {
  size_t pf = 0, cc = 0;
  for (int i = 0; i < a.count; ++i) {
    if (a.d[i].parts > 1) {
      const size_t tiles = static_cast<size_t>(a.d[i].n + 31) / 32 * ((a.m + 31) / 32);
      pf += tiles * a.d[i].parts * 1024;
      cc += tiles;
    }
  }
  *partial_floats = pf;
  *counters = cc;
}

void bind_skinny(SkinnyArgs& a, float* partial, int* counters) {
  for (int i = 0; i < a.count; ++i) {
    SkinnyDesc& d = a.d[i];
    if (d.parts > 1) {
      const size_t tiles = static_cast<size_t>(d.n + 31) / 32 * ((a.m + 31) / 32);
      d.partial = partial;
      d.counters = counters;
      partial += tiles * d.parts * 1024;
      counters += tiles;
    }
  }
}

void launch_gemm_skinny(bool w8, const SkinnyArgs& a, int blocks, hipStream_t stream) {
  const bool pair = a.d[0].w2 != nullptr;
  const int kw = a.waves;
  if (w8) {
    if (pair) {
      launch_skinny_kw<true, true>(a, blocks, kw, stream);
    } else {
      launch_skinny_kw<true, false>(a, blocks, kw, stream);
    }
  } else {
    if (pair) {
      launch_skinny_kw<false, true>(a, blocks, kw, stream);
    } else {
      launch_skinny_kw<false, false>(a, blocks, kw, stream);
    }
  }
}

int gemm_pick_tile(int m, int n) {
  // A single GEMM at the Qwen shapes (M <= 512) gives too few 256 x 128
  // tiles to fill the 256 CUs, so the 64 x 64 tile (the most workgroups, up
  // to 4 per CU) is fastest there; once the wide tile alone has a workgroup
  // for (nearly) every CU, its lower LDS traffic per FLOP wins.
  const long long wide = static_cast<long long>((m + kWideRows - 1) / kWideRows) *
                         ((n + kWideCols - 1) / kWideCols);
  if (m >= kWideRows && wide >= 240) return kGemmTile256x128;
  return kGemmTile64x64;
}

int gemm_tile_rows(int tile) {
  static const int rows[kGemmTileCount] = {128, 128, 64, 64, 32, kWideRows};
  return rows[tile];
}

int gemm_tile_cols(int tile) {
  static const int cols[kGemmTileCount] = {128, 64, 128, 64, 128, kWideCols};
  return cols[tile];
}

void launch_gemm_grouped(int tile, bool w8, const GemmGroupDesc* device_descs, int count,
                         int total_blocks, hipStream_t stream) {
  const dim3 grid(total_blocks), block(kThreads);
  if (tile == kGemmTile128x128) {
    if (w8) {
      hipLaunchKernelGGL((gemm_grouped_kernel<128, 128, 2, true>), grid, block, 0, stream,
                         device_descs, count);
    } else {
      hipLaunchKernelGGL((gemm_grouped_kernel<128, 128, 2, false>), grid, block, 0, stream,
                         device_descs, count);
    }
  } else if (w8) {
    hipLaunchKernelGGL((gemm_grouped_kernel<64, 64, 2, true>), grid, block, 0, stream,
                       device_descs, count);
  } else {
    hipLaunchKernelGGL((gemm_grouped_kernel<64, 64, 2, false>), grid, block, 0, stream,
                       device_descs, count);
  }
}

void launch_gemm_wide_grouped(bool w8, const GemmGroupDesc* descs, int count, int units,
                              const WideBlockMap& gmap, const SplitReduceDesc* rdescs, int rcount,
                              int reducers, const ReduceBlockMap& rmap, hipStream_t stream) {
  if (w8) {
    hipLaunchKernelGGL((gemm_wide_grouped_kernel<true>), dim3(units), dim3(kWideThreads), 0, stream,
                       descs, count, gmap);
  } else {
    hipLaunchKernelGGL((gemm_wide_grouped_kernel<false>), dim3(units), dim3(kWideThreads), 0,
                       stream, descs, count, gmap);
  }
  if (rcount > 0) {
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(reducers), dim3(256), 0, stream, rdescs, rcount,
                       rmap);
  }
}

void launch_gemm_wide_grouped_timeline(bool w8, const GemmGroupDesc* descs, int count, int units,
                                       const WideBlockMap& gmap, unsigned long long* stamps,
                                       const SplitReduceDesc* rdescs, int rcount, int reducers,
                                       const ReduceBlockMap& rmap, hipStream_t stream) {
  if (w8) {
    hipLaunchKernelGGL((gemm_wide_grouped_timeline_kernel<true>), dim3(units), dim3(kWideThreads),
                       0, stream, descs, count, gmap, stamps);
  } else {
    hipLaunchKernelGGL((gemm_wide_grouped_timeline_kernel<false>), dim3(units), dim3(kWideThreads),
                       0, stream, descs, count, gmap, stamps);
  }
  if (rcount > 0) {
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(reducers), dim3(256), 0, stream, rdescs, rcount,
                       rmap);
  }
}

void launch_gemm_wide_grouped_timeline(const GemmGroupLaunch& l, unsigned long long* stamps,
                                       hipStream_t stream) {
  if (l.w8) {
    hipLaunchKernelGGL((gemm_wide_inline_timeline_kernel<true>), dim3(l.blocks),
                       dim3(kWideThreads), 0, stream, l.g, l.gmap, stamps);
  } else {
    hipLaunchKernelGGL((gemm_wide_inline_timeline_kernel<false>), dim3(l.blocks),
                       dim3(kWideThreads), 0, stream, l.g, l.gmap, stamps);
  }
  if (l.r.count > 0) {
    hipLaunchKernelGGL(splitk_reduce_inline_kernel, dim3(l.reducers), dim3(256), 0, stream, l.r,
                       l.rmap);
  }
}

void launch_gemm_group_inline(const GemmGroupLaunch& l, hipStream_t stream) {
  const dim3 grid(l.blocks);
  if (l.tile == kGemmTile256x128) {
    if (l.w8) {
      hipLaunchKernelGGL((gemm_wide_inline_kernel<true>), grid, dim3(kWideThreads), 0, stream,
                         l.g, l.gmap);
    } else {
      hipLaunchKernelGGL((gemm_wide_inline_kernel<false>), grid, dim3(kWideThreads), 0, stream,
                         l.g, l.gmap);
    }
    if (l.r.count > 0) {
      hipLaunchKernelGGL(splitk_reduce_inline_kernel, dim3(l.reducers), dim3(256), 0, stream,
                         l.r, l.rmap);
    }
  } else if (l.tile == kGemmTile128x128) {
    if (l.w8) {
      hipLaunchKernelGGL((gemm_grouped_inline_kernel<128, 128, 2, true>), grid, dim3(kThreads),
                         0, stream, l.g);
    } else {
      hipLaunchKernelGGL((gemm_grouped_inline_kernel<128, 128, 2, false>), grid, dim3(kThreads),
                         0, stream, l.g);
    }
  } else if (l.w8) {
    hipLaunchKernelGGL((gemm_grouped_inline_kernel<64, 64, 2, true>), grid, dim3(kThreads), 0,
                       stream, l.g);
  } else {
    hipLaunchKernelGGL((gemm_grouped_inline_kernel<64, 64, 2, false>), grid, dim3(kThreads), 0,
                       stream, l.g);
  }
}

bool gate_up_silu_supported(const void* gate_w, const void* up_w, const uint16_t* x, int m,
                            int inter, int hidden) {
  return m > 0 && inter > 0 && gemm_mfma_supported(gate_w, x, m, inter, hidden) &&
         gemm_mfma_supported(up_w, x, m, inter, hidden);
}

void launch_gate_up_silu(bool w8, const void* gate_w, const uint16_t* gate_s,
                         const uint16_t* gate_b, const void* up_w, const uint16_t* up_s,
                         const uint16_t* up_b, const uint16_t* x, uint16_t* y, int m, int inter,
                         int hidden, hipStream_t stream) {
  GemmGroupLaunch l{};
  GemmGroupDesc& d = l.g.d[0];
  d = GemmGroupDesc{gate_w, gate_s, gate_b, x, y, m, 2 * inter, hidden, 0, 0, 1, hidden / kStageK,
                    nullptr, nullptr, up_w, up_s, up_b};
  d.tiles_m = (m + kWideRows - 1) / kWideRows;
  l.g.count = 1;
  l.w8 = w8;
  l.tile = kGemmTile256x128;
  l.blocks = d.tiles_m * ((inter + kWideCols / 2 - 1) / (kWideCols / 2));
  launch_gemm_group_inline(l, stream);
}

void launch_gemm_mfma(int tile, bool w8, const GemmArgs& a, hipStream_t stream) {
  if (w8) {
    launch_config<true>(tile, a, stream);
  } else {
    launch_config<false>(tile, a, stream);
  }
}

}  // namespace qlin

// ================================================================ C ABI ==

using namespace qlin;

namespace {

// ---- lone GEMMs with a caller workspace ----
// The layout of a lone call: the one-GEMM group of the prefill's inline
// launches (layout_gemm_group with fill), so its split rule is theirs.  In
// the workspace the split tiles' arrival counters start at its beginning,
// counter t at int t, and the FP32 partial tiles end (256-byte aligned) at
// its end.  So counter t has one address for every call on the workspace,
// and as long as the workspace covers the largest partials plus the most
// counters of the calls made on it (what infer_hip_gemm_workspace_bytes
// returns), no call's partials overwrite a counter, which every call
// leaves at zero.
// Calls of at most kSkinnyMaxTokens tokens run the skinny kernel, split over
// K into workgroups (long K) on the same workspace layout.
struct LoneLayout {
  GemmGroupLaunch l{};
  bool skinny = false;
  SkinnyArgs sk{};
  int sk_blocks = 0;
  size_t partial_bytes = 0;  // 0: no split
  size_t counter_bytes = 0;
};

size_t round256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

int current_cus(int* cus) {
  int device = 0;
  hipError_t st = hipGetDevice(&device);
  if (st == hipSuccess) {
    st = hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, device);
  }
  if (st != hipSuccess || *cus <= 0) {
    (void)hipGetLastError();
    return fail(INFER_HIP_RUNTIME_ERROR, "gemm workspace: no device to lay the call out for");
  }
  return INFER_HIP_OK;
}

LoneLayout lone_layout(bool w8, const void* w, const uint16_t* s, const uint16_t* bias,
                       const uint16_t* x, uint16_t* y, int m, int n, int k, int cus) {
  LoneLayout o;
  if (m >= 2 && gemm_skinny_supported(w, x, m, n, k) && gemm_skinny_preferred(w8, m, n, k)) {
    o.skinny = true;
    o.sk.count = 1;
    o.sk.m = m;
    o.sk.d[0] = SkinnyDesc{w, w8 ? s : nullptr, bias, nullptr, nullptr, nullptr, x, y, n, k, 0};
    o.sk_blocks = layout_skinny(o.sk, true);
    size_t pf = 0, cc = 0;
    skinny_scratch(o.sk, &pf, &cc);
    if (pf > 0) {
      o.partial_bytes = round256(pf * sizeof(float));
      o.counter_bytes = round256(cc * sizeof(int));
    }
    return o;
  }
  GemmGroupDesc& d = o.l.g.d[0];
  d = GemmGroupDesc{w, s, bias, x, y, m, n, k, 0, 0, 1, k / kStageK, nullptr, nullptr};
  size_t pf = 0, cc = 0;
  o.l.tile = layout_gemm_group(&d, 1, cus, true, &o.l.blocks, &pf, &cc);
  o.l.g.count = 1;
  o.l.w8 = w8;
  if (d.splits > 1) {
    o.partial_bytes = round256(pf * sizeof(float));
    o.counter_bytes = round256(cc * sizeof(int));
  }
  return o;
}

// Runs a lone call split over K on the workspace; *done is false when the
// call does not split (the caller then takes the plain path).
int launch_lone_split(bool w8, const void* w, const uint16_t* s, const uint16_t* bias,
                      const uint16_t* x, uint16_t* y, int m, int n, int k, void* ws,
                      size_t ws_bytes, hipStream_t stream, bool* done) {
  *done = false;
  int cus = 0;
  const int rc = current_cus(&cus);
  if (rc != INFER_HIP_OK) return rc;
  LoneLayout o = lone_layout(w8, w, s, bias, x, y, m, n, k, cus);
  if (o.partial_bytes == 0 || (!o.skinny && o.l.blocks <= 0)) return INFER_HIP_OK;
  if (!ws) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "gemm: this call splits K and needs a workspace of %zu bytes (none given)",
                o.partial_bytes + o.counter_bytes + 256);
  }
  if (!aligned16(ws)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemm: the workspace must be 16-byte aligned");
  }
  const uintptr_t begin = reinterpret_cast<uintptr_t>(ws);
  const uintptr_t end = begin + ws_bytes;
  const uintptr_t pbase =
      ws_bytes >= o.partial_bytes ? (end - o.partial_bytes) & ~static_cast<uintptr_t>(255) : 0;
  if (ws_bytes < o.partial_bytes || pbase < begin + o.counter_bytes) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "gemm: this call splits K and needs a workspace of %zu bytes (%zu given)",
                o.partial_bytes + o.counter_bytes + 256, ws_bytes);
  }
  int* counters = static_cast<int*>(ws);
  float* partial = reinterpret_cast<float*>(pbase);
  if (o.skinny) {
    bind_skinny(o.sk, partial, counters);
    launch_gemm_skinny(w8, o.sk, o.sk_blocks, stream);
  } else {
    o.l.r.count = bind_gemm_group(o.l.g.d, 1, o.l.tile, partial, counters, o.l.r.d,
                                  &o.l.reducers);
    launch_gemm_group_inline(o.l, stream);
  }
  *done = true;
  return INFER_HIP_OK;
}

// ws_mode: the caller passed a workspace (the _ws entry points).
// A lone GEMM of at most kSkinnyMaxTokens tokens without a workspace: one
// skinny launch, K split only over each workgroup's waves.
void launch_lone_skinny(bool w8, const void* weight, const uint16_t* scales,
                        const uint16_t* bias, const uint16_t* input, uint16_t* output, int tokens,
                        int n, int k, hipStream_t stream) {
  SkinnyArgs a{};
  a.count = 1;
  a.m = tokens;
  a.d[0] = SkinnyDesc{weight, w8 ? scales : nullptr, bias, nullptr, nullptr, nullptr, input,
                      output, n, k, 0};
  const int blocks = layout_skinny(a, false);
  launch_gemm_skinny(w8, a, blocks, stream);
}

int gemm_w8a16_impl(const int8_t* weight, const uint16_t* scales, int group_size,
                    const uint16_t* bias, const uint16_t* input, uint16_t* output, int tokens,
                    int out_features, int in_features, int tile, hipStream_t stream,
                    bool ws_mode = false, void* ws = nullptr, size_t ws_bytes = 0) {
  // kernels.cu:1661 — the only supported group size.
  if (group_size != 64) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "w8a16 group size must be 64 (got %d)", group_size);
  }
  if (tokens <= 0 || out_features <= 0 || in_features < 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemm_w8a16: bad shape M=%d N=%d K=%d", tokens,
                out_features, in_features);
  }
  if (tile < -1 || tile >= kGemmTileCount) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemm_w8a16: no tile %d", tile);
  }
  if (!output || (in_features > 0 && (!weight || !scales || !input))) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemm_w8a16: null required pointer");
  }
  if (tokens == 1 && w8a16_gemv_fast_supported(weight, input, in_features)) {
    launch_w8a16_gemv_fast({weight, scales, bias, input, output, out_features, in_features},
                           stream);
  } else if (tile < 0 && tokens > 1 &&
             gemm_skinny_supported(weight, input, tokens, out_features, in_features) &&
             gemm_skinny_preferred(true, tokens, out_features, in_features)) {
    bool done = false;
    if (ws_mode) {  // long K: split over workgroups on the workspace
      const int rc = launch_lone_split(true, weight, scales, bias, input, output, tokens,
                                       out_features, in_features, ws, ws_bytes, stream, &done);
      if (rc != INFER_HIP_OK) return rc;
    }
    if (!done) {
      launch_lone_skinny(true, weight, scales, bias, input, output, tokens, out_features,
                         in_features, stream);
    }
  } else if (tokens > 1 && gemm_mfma_supported(weight, input, tokens, out_features, in_features)) {
    bool done = false;
    if (ws_mode) {
      const int rc = launch_lone_split(true, weight, scales, bias, input, output, tokens,
                                       out_features, in_features, ws, ws_bytes, stream, &done);
      if (rc != INFER_HIP_OK) return rc;
    }
    if (!done) {
      const GemmArgs a{weight, scales, bias, input, output, tokens, out_features, in_features};
      launch_gemm_mfma(tile < 0 ? gemm_pick_tile(tokens, out_features) : tile, true, a, stream);
    }
  } else {
    launch_w8a16_linear_generic(weight, scales, group_size, bias, input, output, tokens,
                                out_features, in_features, stream);
  }
  return check_launch("gemm_w8a16");
}

int gemm_bf16_impl(const uint16_t* weight, const uint16_t* bias, const uint16_t* input,
                   uint16_t* output, int tokens, int out_features, int in_features, int tile,
                   hipStream_t stream, bool ws_mode = false, void* ws = nullptr,
                   size_t ws_bytes = 0) {
  if (tokens <= 0 || out_features <= 0 || in_features < 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemm_bf16: bad shape M=%d N=%d K=%d", tokens,
                out_features, in_features);
  }
  if (tile < -1 || tile >= kGemmTileCount) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemm_bf16: no tile %d", tile);
  }
  if (!output || (in_features > 0 && (!weight || !input))) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemm_bf16: null required pointer");
  }
  if (tokens == 1 && bf16_gemv_fast_supported(weight, input, in_features)) {
    launch_bf16_gemv_fast({weight, bias, input, output, out_features, in_features}, stream);
  } else if (tile < 0 && tokens > 1 &&
             gemm_skinny_supported(weight, input, tokens, out_features, in_features) &&
             gemm_skinny_preferred(false, tokens, out_features, in_features)) {
    bool done = false;
    if (ws_mode) {  // long K: split over workgroups on the workspace
      const int rc = launch_lone_split(false, weight, nullptr, bias, input, output, tokens,
                                       out_features, in_features, ws, ws_bytes, stream, &done);
      if (rc != INFER_HIP_OK) return rc;
    }
    if (!done) {
      launch_lone_skinny(false, weight, nullptr, bias, input, output, tokens, out_features,
                         in_features, stream);
    }
  } else if (tokens > 1 && gemm_mfma_supported(weight, input, tokens, out_features, in_features)) {
    bool done = false;
    if (ws_mode) {
      const int rc = launch_lone_split(false, weight, nullptr, bias, input, output, tokens,
                                       out_features, in_features, ws, ws_bytes, stream, &done);
      if (rc != INFER_HIP_OK) return rc;
    }
    if (!done) {
      const GemmArgs a{weight, nullptr, bias, input, output, tokens, out_features, in_features};
      launch_gemm_mfma(tile < 0 ? gemm_pick_tile(tokens, out_features) : tile, false, a, stream);
    }
  } else {
    launch_bf16_linear_generic(weight, bias, input, output, tokens, out_features, in_features,
                               stream);
  }
  return check_launch("gemm_bf16");
}

int gate_up_silu_impl(bool w8, const void* gate_w, const uint16_t* gate_s,
                      const uint16_t* gate_b, const void* up_w, const uint16_t* up_s,
                      const uint16_t* up_b, int group_size, const uint16_t* input,
                      uint16_t* output, int tokens, int inter, int hidden, hipStream_t stream) {
  const char* what = w8 ? "gemm_gate_up_silu_w8a16" : "gemm_gate_up_silu_bf16";
  if (w8 && group_size != 64) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "w8a16 group size must be 64 (got %d)", group_size);
  }
  if (tokens <= 0 || inter <= 0 || hidden <= 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: bad shape M=%d intermediate=%d hidden=%d", what,
                tokens, inter, hidden);
  }
  if (!gate_w || !up_w || !input || !output || (w8 && (!gate_s || !up_s))) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "%s: null required pointer", what);
  }
  if (!gate_up_silu_supported(gate_w, up_w, input, tokens, inter, hidden)) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "%s: needs hidden %% 64 == 0, 16-byte aligned weights and input, and operands "
                "under 2 GiB",
                what);
  }
  if (gemm_skinny_preferred(w8, tokens, 2 * inter, hidden)) {  // the pair: two GEMMs' rows
    SkinnyArgs a{};
    a.count = 1;
    a.m = tokens;
    a.d[0] = SkinnyDesc{gate_w, w8 ? gate_s : nullptr, gate_b, up_w, w8 ? up_s : nullptr, up_b,
                        input, output, inter, hidden, 0};
    const int blocks = layout_skinny(a, false);  // a pair is never split
    launch_gemm_skinny(w8, a, blocks, stream);
  } else {
    launch_gate_up_silu(w8, gate_w, gate_s, gate_b, up_w, up_s, up_b, input, output, tokens,
                        inter, hidden, stream);
  }
  return check_launch(what);
}

}  // namespace

extern "C" int infer_hip_gemm_gate_up_silu_w8a16(
    const int8_t* gate_weight, const uint16_t* gate_scales, const uint16_t* gate_bias,
    const int8_t* up_weight, const uint16_t* up_scales, const uint16_t* up_bias, int group_size,
    const uint16_t* input, uint16_t* output, int tokens, int intermediate, int hidden,
    hipStream_t stream) {
  return gate_up_silu_impl(true, gate_weight, gate_scales, gate_bias, up_weight, up_scales,
                           up_bias, group_size, input, output, tokens, intermediate, hidden,
                           stream);
}

extern "C" int infer_hip_gemm_gate_up_silu_bf16(const uint16_t* gate_weight,
                                                const uint16_t* gate_bias,
                                                const uint16_t* up_weight,
                                                const uint16_t* up_bias, const uint16_t* input,
                                                uint16_t* output, int tokens, int intermediate,
                                                int hidden, hipStream_t stream) {
  return gate_up_silu_impl(false, gate_weight, nullptr, gate_bias, up_weight, nullptr, up_bias,
                           64, input, output, tokens, intermediate, hidden, stream);
}

extern "C" int infer_hip_gemm_w8a16(const int8_t* weight, const uint16_t* scales,
                                    int group_size, const uint16_t* bias,
                                    const uint16_t* input, uint16_t* output, int tokens,
                                    int out_features, int in_features, hipStream_t stream) {
  return gemm_w8a16_impl(weight, scales, group_size, bias, input, output, tokens, out_features,
                         in_features, -1, stream);
}

extern "C" int infer_hip_gemm_bf16(const uint16_t* weight, const uint16_t* bias,
                                   const uint16_t* input, uint16_t* output, int tokens,
                                   int out_features, int in_features, hipStream_t stream) {
  return gemm_bf16_impl(weight, bias, input, output, tokens, out_features, in_features, -1,
                        stream);
}

extern "C" int infer_hip_gemm_tile_count(void) { return kGemmTileCount; }

extern "C" size_t infer_hip_gemm_workspace_bytes(int max_tokens, int out_features,
                                                 int in_features) {
  if (max_tokens < 2 || out_features <= 0 || in_features < kStageK ||
      in_features % kStageK != 0) {
    return 0;
  }
  int cus = 0;
  if (current_cus(&cus) != INFER_HIP_OK) return 0;
  size_t partials = 0, counters = 0;
  for (int m = 2; m <= max_tokens; ++m) {
    for (const bool w8 : {false, true}) {  // (the two may pick different kernels)
      const LoneLayout o = lone_layout(w8, nullptr, nullptr, nullptr, nullptr, nullptr, m,
                                       out_features, in_features, cus);
      partials = std::max(partials, o.partial_bytes);
      counters = std::max(counters, o.counter_bytes);
    }
  }
  if (partials == 0) return 0;       // no call splits
  return partials + counters + 256;  // 256: the partials' alignment at the end
}

extern "C" int infer_hip_gemm_w8a16_ws(const int8_t* weight, const uint16_t* scales,
                                       int group_size, const uint16_t* bias,
                                       const uint16_t* input, uint16_t* output, int tokens,
                                       int out_features, int in_features, void* workspace,
                                       size_t workspace_bytes, hipStream_t stream) {
  return gemm_w8a16_impl(weight, scales, group_size, bias, input, output, tokens, out_features,
                         in_features, -1, stream, true, workspace, workspace_bytes);
}

extern "C" int infer_hip_gemm_bf16_ws(const uint16_t* weight, const uint16_t* bias,
                                      const uint16_t* input, uint16_t* output, int tokens,
                                      int out_features, int in_features, void* workspace,
                                      size_t workspace_bytes, hipStream_t stream) {
  return gemm_bf16_impl(weight, bias, input, output, tokens, out_features, in_features, -1,
                        stream, true, workspace, workspace_bytes);
}

extern "C" int infer_hip_gemm_w8a16_tile(const int8_t* weight, const uint16_t* scales,
                                         int group_size, const uint16_t* bias,
                                         const uint16_t* input, uint16_t* output, int tokens,
                                         int out_features, int in_features, int tile,
                                         hipStream_t stream) {
  return gemm_w8a16_impl(weight, scales, group_size, bias, input, output, tokens, out_features,
                         in_features, tile, stream);
}

extern "C" int infer_hip_gemm_bf16_tile(const uint16_t* weight, const uint16_t* bias,
                                        const uint16_t* input, uint16_t* output, int tokens,
                                        int out_features, int in_features, int tile,
                                        hipStream_t stream) {
  return gemm_bf16_impl(weight, bias, input, output, tokens, out_features, in_features, tile,
                        stream);
}
