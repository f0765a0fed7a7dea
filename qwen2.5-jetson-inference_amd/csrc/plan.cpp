// Grouped plans: many independent GEMVs (decode) or GEMMs (prefill) run by
// one launch from a descriptor table resolved once and kept in device memory.
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

// ---------------------------------------------------------------------------
// Grouped GEMM plans (prefill): many independent GEMMs in one launch of the
// MFMA kernel, one workgroup per output tile (or part of one, split over K).

namespace qlin {

namespace {
constexpr int kWideRowsHost = 256;  // gemm_tile_rows(kGemmTile256x128)
constexpr int kWideColsHost = 128;
}  // namespace

// 128 x 128 tiles for a lone long-K GEMM (a measured alternative, off by
// default; see linear_kernels.hpp).
#ifndef QLIN_GROUP_TILE128
#define QLIN_GROUP_TILE128 0
#endif
int layout_gemm_group(GemmGroupDesc* table, int count, int cus, bool fill, int* blocks_out,
                      size_t* partial_floats, size_t* counters) {
  int min_tokens = table[0].m;
  long long wide_tiles = 0;
  for (int i = 0; i < count; ++i) {
    min_tokens = std::min(min_tokens, table[i].m);
    wide_tiles += static_cast<long long>((table[i].m + kWideRowsHost - 1) / kWideRowsHost) *
                  ((table[i].n + kWideColsHost - 1) / kWideColsHost);
  }
  // Once every GEMM has 256 rows or more, the 8-wave 256 x 128 tile: it
  // moves the fewest LDS bytes per FLOP and runs two waves per SIMD.  Below
  // that, 64 x 64 tiles (the most workgroups; up to 4 per CU).  A `fill`
  // group also needs wide tiles for at least half the CUs: measured on
  // MI355X at M = 512, q|k|v (18 wide tiles) and o (14) take 7.9 us on 64 x 64
  // tiles against 15-18 us on wide ones, while gate|up (152 wide tiles) takes
  // 18.3 us wide against 20.9 us.
  const bool wide = min_tokens >= kWideRowsHost && (!fill || 2 * wide_tiles >= cus);
  int tile = wide ? kGemmTile256x128 : kGemmTile64x64;
  const bool t128 = QLIN_GROUP_TILE128 && fill && !wide && count == 1 && min_tokens >= 128 &&
                    table[0].k >= 2048;
  if (t128) tile = kGemmTile128x128;
  const int bm = gemm_tile_rows(tile), bn = gemm_tile_cols(tile);
  int min_stages = 1 << 30, max_stages = 0;
  for (int i = 0; i < count; ++i) {
    GemmGroupDesc& d = table[i];
    d.tiles_m = (d.m + bm - 1) / bm;
    d.splits = 1;
    d.split_stages = d.k / 64;
    d.partial = nullptr;
    d.counters = nullptr;
    min_stages = std::min(min_stages, d.k / 64);
    max_stages = std::max(max_stages, d.k / 64);
  }
  auto units_for = [&](int t) {
    long long u = 0;
    for (int i = 0; i < count; ++i) {
      const GemmGroupDesc& d = table[i];
      const int stages = d.k / 64;
      const int per = (stages + ((stages + t - 1) / t) - 1) / ((stages + t - 1) / t);
      const int parts = (stages + per - 1) / per;
      u += static_cast<long long>(d.tiles_m) * ((d.n + bn - 1) / bn) * parts;
    }
    return u;
  };
  // Split K so that no unit is much longer than the group's shortest
  // reduction (at least 8 stages of 64): a lone long-K tile would otherwise
  // be the whole launch's critical path.  With the wide tile every CU holds
  // one workgroup, so the unit length is raised, if needed, until all units
  // fit on the CUs at once (M = 512 layer: down's 76 stages in 5 parts of 16
  // instead of 6 of 13, 254 units on 256 CUs).
  // A `fill` group is split into at most 4 parts of at least 14 stages, and
  // into fewer while it has more than two units per CU: measured at
  // M = 128-512, down (76 stages) is fastest in 4 parts of 19 on 64 x 64
  // tiles (16.2 us at M = 512, 448 units), and 14-stage GEMMs gain nothing
  // from a split.
  // A 64 x 64 plan likewise raises the part length until its units fit two
  // per CU: at M = 128 a layer's 7 GEMMs (368 whole tiles) with down in 5
  // parts of 16 (508 units) take 15.8 us against 18.5 us with 6 parts of 13
  // (536 units, the last 24 in a second round).  Shorter parts lose: at
  // M = 32, 2-4 stage parts of every GEMM take 19.4 us against 13.8 us,
  // their in-kernel hand-offs costing more than the shorter chains save.
  int target = std::max(8, min_stages);
  if (t128) {
    target = (max_stages + 7) / 8;  // 8 parts
  } else if (fill) {
    target = std::min(max_stages, std::max(14, (max_stages + 3) / 4));
    while (target < max_stages && units_for(target) > 2ll * cus) ++target;
  } else if (tile == kGemmTile256x128) {
    while (target < max_stages && units_for(target) > cus) ++target;
    target = std::max(target, (max_stages + kWideMaxParts - 1) / kWideMaxParts);
  } else {
    while (target < max_stages && units_for(target) > 2ll * cus) ++target;
  }
  // arrival counters per split tile: the 64 x 64 tiles' last-arrival count;
  // the wide tile's in-launch hand-off (or none with a reduction launch)
  const size_t counter_ints =
      tile != kGemmTile256x128
          ? 1
          : (QLIN_WIDE_INKERNEL ? kWideSplitCounterInts : (QLIN_WIDE_HELP ? kHelpCounterInts : 0));
  size_t pf = 0, cc = 0;
  for (int i = 0; i < count; ++i) {
    GemmGroupDesc& d = table[i];
    const int stages = d.k / 64;
    const int parts = (stages + target - 1) / target;
    if (parts > 1) {
      d.split_stages = (stages + parts - 1) / parts;
      d.splits = (stages + d.split_stages - 1) / d.split_stages;  // no empty part
      const size_t tiles = static_cast<size_t>(d.tiles_m) * ((d.n + bn - 1) / bn);
      pf += tiles * d.splits * bm * bn;
      cc += tiles * counter_ints;
    }
  }
  // Longest units first: they take longest, so starting them earliest
  // shortens the launch's tail.
  std::stable_sort(table, table + count, [](const GemmGroupDesc& a, const GemmGroupDesc& b) {
    return a.split_stages > b.split_stages;
  });
  long long blocks = 0;
  for (int i = 0; i < count; ++i) {
    GemmGroupDesc& d = table[i];
    d.block_begin = static_cast<int>(blocks);
    blocks += static_cast<long long>(d.tiles_m) * ((d.n + bn - 1) / bn) * d.splits;
  }
  *blocks_out = blocks > 0x7FFFFFFF ? -1 : static_cast<int>(blocks);
  *partial_floats = pf;
  *counters = cc;
  return tile;
}

int bind_gemm_group(GemmGroupDesc* table, int count, int tile, float* partial, int* counters,
                    SplitReduceDesc* reduce, int* reducers) {
  const bool wide = tile == kGemmTile256x128;
  const int bm = gemm_tile_rows(tile), bn = gemm_tile_cols(tile);
  size_t pf = 0, cc = 0;
  int rcount = 0, rblocks = 0;
  for (int i = 0; i < count; ++i) {
    GemmGroupDesc& d = table[i];
    if (d.splits <= 1) continue;
    const size_t tiles = static_cast<size_t>(d.tiles_m) * ((d.n + bn - 1) / bn);
    d.partial = partial + pf;
    if (!wide) {
      d.counters = counters + cc;
      cc += tiles;
    } else if (QLIN_WIDE_INKERNEL) {
      d.counters = counters + cc;
      cc += tiles * kWideSplitCounterInts;
    } else {
      if (QLIN_WIDE_HELP) {  // the reduction launch stays for unmapped launches
        d.counters = counters + cc;
        cc += tiles * kHelpCounterInts;
      }
      reduce[rcount++] =
          SplitReduceDesc{d.partial, d.bias, d.y, d.m, d.n, d.tiles_m, d.splits, rblocks};
      rblocks += static_cast<int>(tiles) * (bm / kSplitReduceRows);
    }
    pf += tiles * d.splits * bm * bn;
  }
  *reducers = rblocks;
  return rcount;
}

void map_wide_group_to_xcds(const GemmGroupDesc* table, int count, int blocks, WideBlockMap* gmap,
                            ReduceBlockMap* rmap, int* reducers) {
  *gmap = WideBlockMap{};
  *rmap = ReduceBlockMap{};
  constexpr int kBlocksPerTile = kWideRowsHost / kSplitReduceRows;
  int split_tiles = 0;
  for (int i = 0; i < count; ++i) {
    if (table[i].splits > 1) {
      split_tiles += table[i].tiles_m * ((table[i].n + kWideColsHost - 1) / kWideColsHost);
    }
  }
  *reducers = QLIN_WIDE_INKERNEL ? 0 : split_tiles * kBlocksPerTile;
#if !QLIN_XCD_MAP
  return;
#endif
  if (split_tiles == 0 || blocks <= 0 || blocks > kWideMapBlocks) return;
  // XCD x runs the workgroups b < blocks with b % 8 == x.
  int cap[kXcds];
  for (int x = 0; x < kXcds; ++x) cap[x] = x < blocks ? (blocks - x + kXcds - 1) / kXcds : 0;
  std::vector<int> on[kXcds];         // logical blocks placed on each XCD
  std::vector<int> tiles_on[kXcds];   // split tiles (numbered over the plan) on each XCD
  int tile_id = 0;
  for (int i = 0; i < count; ++i) {
    const GemmGroupDesc& d = table[i];
    if (d.splits <= 1) continue;
    const int tiles = d.tiles_m * ((d.n + kWideColsHost - 1) / kWideColsHost);
    for (int t = 0; t < tiles; ++t, ++tile_id) {
      int best = -1;
      for (int x = 0; x < kXcds; ++x) {
        const int free = cap[x] - static_cast<int>(on[x].size());
        if (free >= d.splits && (best < 0 || free > cap[best] - static_cast<int>(on[best].size()))) {
          best = x;
        }
      }
      if (best < 0) return;  // unmapped
      for (int p = 0; p < d.splits; ++p) on[best].push_back(d.block_begin + t * d.splits + p);
      tiles_on[best].push_back(tile_id);
    }
  }
  // whole tiles fill the remaining workgroups, XCD by XCD
  int x = 0;
  for (int i = 0; i < count; ++i) {
    const GemmGroupDesc& d = table[i];
    if (d.splits > 1) continue;
    const int units = d.tiles_m * ((d.n + kWideColsHost - 1) / kWideColsHost);
    for (int u = 0; u < units; ++u) {
      while (static_cast<int>(on[x].size()) >= cap[x]) ++x;  // capacities sum to blocks
      on[x].push_back(d.block_begin + u);
    }
  }
  int slots = 0;
  for (int y = 0; y < kXcds; ++y) slots = std::max(slots, static_cast<int>(tiles_on[y].size()));
  for (int y = 0; y < kXcds; ++y) {
    for (size_t k = 0; k < on[y].size(); ++k) {
      gmap->logical[k * kXcds + y] = static_cast<uint8_t>(on[y][k]);
    }
  }
  gmap->mapped = 1;
  if (QLIN_WIDE_HELP && !QLIN_WIDE_INKERNEL && slots <= kHelpTiles && tile_id <= 0xFE) {
    for (int y = 0; y < kXcds; ++y) {
      for (int k = 0; k < kHelpTiles; ++k) {
        gmap->help_tiles[y][k] =
            k < static_cast<int>(tiles_on[y].size()) ? static_cast<uint8_t>(tiles_on[y][k]) : 0xFF;
      }
      // the whole-tile workgroups of XCD y sum its split tiles' slices
      int helpers = 0;
      for (size_t k = 0; k < on[y].size(); ++k) {
        const int logical = on[y][k];
        bool part = false;
        for (int i = 0; i < count; ++i) {
          const GemmGroupDesc& d = table[i];
          const int units = d.tiles_m * ((d.n + kWideColsHost - 1) / kWideColsHost) * d.splits;
          if (logical >= d.block_begin && logical < d.block_begin + units) part = d.splits > 1;
        }
        gmap->help_rank[k * kXcds + y] = part ? 0xFF : static_cast<uint8_t>(helpers++);
      }
      gmap->help_members[y] = static_cast<uint8_t>(helpers);
    }
    gmap->help = 1;
    *reducers = 0;
    return;
  }
  if (QLIN_WIDE_INKERNEL || slots > kReduceSlots || tile_id > 0xFE) return;  // reduction unmapped
  for (int y = 0; y < kXcds; ++y) {
    for (int k = 0; k < kReduceSlots; ++k) {
      rmap->tile[y][k] =
          k < static_cast<int>(tiles_on[y].size()) ? static_cast<uint8_t>(tiles_on[y][k]) : 0xFF;
    }
  }
  rmap->slots = slots;
  *reducers = kXcds * slots * kBlocksPerTile;
}

}  // namespace qlin

struct infer_hip_gemm_plan {
  GemmGroupDesc* table = nullptr;  // device memory
  float* partial = nullptr;        // split-K partial tiles (device)
  int* counters = nullptr;         // split-K arrival counters (device, zeroed)
  SplitReduceDesc* reduce = nullptr;  // split-K reduction table (device; wide tile)
  WideBlockMap block_map;             // wide tile: workgroup -> unit
  ReduceBlockMap reduce_map;          // wide tile: workgroup -> reduction block
  // A wide-tile plan of at most kInlineGroupMax GEMMs launches with its
  // descriptors in the kernel arguments: no dependent reads of the table
  // before a workgroup's first loads.
  bool inline_wide = false;
  GemmGroupLaunch wide_launch{};
  int reduce_count = 0;
  int reduce_blocks = 0;
  int count = 0;
  int blocks = 0;
  int device = 0;
  int tile = kGemmTile64x64;
  bool w8 = false;
  double flops = 0.0;
  // A plan of at most kSkinnyMaxDescs GEMMs of one token count where the
  // skinny kernel is preferred for every one of them runs as one skinny
  // launch (no table; scratch only for K parts).
  bool skinny = false;
  SkinnyArgs skinny_args{};
};

extern "C" int infer_hip_gemm_plan_create(const infer_hip_gemm_desc* descs, int count,
                                          infer_hip_gemm_plan** plan_out) {
  if (!plan_out) return fail(INFER_HIP_INVALID_ARGUMENT, "gemm plan: null output pointer");
  *plan_out = nullptr;
  if (!descs || count <= 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemm plan: need at least one descriptor");
  }
  const bool w8 = descs[0].w8a16 != 0;
  std::vector<GemmGroupDesc> table;
  table.reserve(count);
  double flops = 0.0;
  for (int i = 0; i < count; ++i) {
    const infer_hip_gemm_desc& d = descs[i];
    if ((d.w8a16 != 0) != w8) {
      return fail(INFER_HIP_INVALID_ARGUMENT,
                  "gemm plan: descriptor %d: all descriptors must share one weight type", i);
    }
    if (w8 && d.group_size != 64) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "gemm plan: descriptor %d: group size must be 64",
                  i);
    }
    if (d.tokens < 2 || d.out_features <= 0 || d.in_features <= 0) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "gemm plan: descriptor %d: bad shape M=%d N=%d K=%d",
                  i, d.tokens, d.out_features, d.in_features);
    }
    if (!d.weight || (w8 && !d.scales) || !d.input || !d.output) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "gemm plan: descriptor %d: null pointer", i);
    }
    if (!gemm_mfma_supported(d.weight, d.input, d.tokens, d.out_features, d.in_features)) {
      return fail(INFER_HIP_INVALID_ARGUMENT,
                  "gemm plan: descriptor %d needs K %% 64 == 0, 16-byte aligned weight and "
                  "input and operands under 2 GiB (K=%d)",
                  i, d.in_features);
    }
    table.push_back(GemmGroupDesc{d.weight, w8 ? d.scales : nullptr, d.bias, d.input, d.output,
                                  d.tokens, d.out_features, d.in_features, 0, 0, 1,
                                  d.in_features / 64, nullptr, nullptr});
    flops += 2.0 * d.tokens * d.out_features * d.in_features;
  }
  int device = 0, cus = 0;
  if (hipGetDevice(&device) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) {
    return fail(INFER_HIP_RUNTIME_ERROR, "gemm plan: cannot query the device");
  }
  bool skinny = count <= kSkinnyMaxDescs;
  for (int i = 0; i < count && skinny; ++i) {
    skinny = descs[i].tokens == descs[0].tokens &&
             gemm_skinny_supported(descs[i].weight, descs[i].input, descs[i].tokens,
                                   descs[i].out_features, descs[i].in_features) &&
             gemm_skinny_preferred(w8, descs[i].tokens, descs[i].out_features,
                                   descs[i].in_features);
  }
  if (skinny) {
    auto* plan = new (std::nothrow) infer_hip_gemm_plan();
    if (!plan) return fail(INFER_HIP_RUNTIME_ERROR, "gemm plan: out of host memory");
    plan->count = count;
    plan->w8 = w8;
    plan->flops = flops;
    plan->device = device;
    plan->skinny = true;
    plan->skinny_args.count = count;
    plan->skinny_args.m = descs[0].tokens;
    for (int i = 0; i < count; ++i) {
      const infer_hip_gemm_desc& d = descs[i];
      plan->skinny_args.d[i] = SkinnyDesc{d.weight, w8 ? d.scales : nullptr, d.bias, nullptr,
                                          nullptr, nullptr, d.input, d.output, d.out_features,
                                          d.in_features, 0};
    }
    plan->blocks = layout_skinny(plan->skinny_args, true);
    size_t pf = 0, cc = 0;
    skinny_scratch(plan->skinny_args, &pf, &cc);
    hipError_t st = hipSuccess;
    if (pf > 0) {
      st = hipMalloc(&plan->partial, pf * sizeof(float));
      if (st == hipSuccess) st = hipMalloc(&plan->counters, cc * sizeof(int));
      if (st == hipSuccess) st = hipMemset(plan->counters, 0, cc * sizeof(int));
      if (st == hipSuccess) bind_skinny(plan->skinny_args, plan->partial, plan->counters);
    }
    if (st != hipSuccess) {
      if (plan->partial) (void)hipFree(plan->partial);
      if (plan->counters) (void)hipFree(plan->counters);
      delete plan;
      return fail(INFER_HIP_RUNTIME_ERROR, "gemm plan: %s", hipGetErrorString(st));
    }
    *plan_out = plan;
    return ok();
  }
  int blocks = 0;
  size_t partial_floats = 0, counter_count = 0;
  const int tile = layout_gemm_group(table.data(), count, cus, false, &blocks, &partial_floats,
                                     &counter_count);
  if (blocks < 0) return fail(INFER_HIP_INVALID_ARGUMENT, "gemm plan: too many tiles");
  auto* plan = new (std::nothrow) infer_hip_gemm_plan();
  if (!plan) return fail(INFER_HIP_RUNTIME_ERROR, "gemm plan: out of host memory");
  plan->count = count;
  plan->blocks = blocks;
  plan->w8 = w8;
  plan->tile = tile;
  plan->flops = flops;
  // Split tiles: with the 64 x 64 tile the last part to arrive (counted on a
  // per-tile counter) sums the parts inside the launch; the wide tile's
  // parts are summed by a second, reduction launch spread over many CUs —
  // one CU reading every part of a 256 x 128 FP32 tile took microseconds.
  std::vector<SplitReduceDesc> reduce(count);
  int rcount = 0;
  hipError_t st = hipGetDevice(&plan->device);
  if (st == hipSuccess && partial_floats > 0) {
    st = hipMalloc(&plan->partial, partial_floats * sizeof(float));
    if (st == hipSuccess && counter_count > 0) {
      st = hipMalloc(&plan->counters, counter_count * sizeof(int));
      if (st == hipSuccess) st = hipMemset(plan->counters, 0, counter_count * sizeof(int));
    }
    if (st == hipSuccess) {
      rcount = bind_gemm_group(table.data(), count, tile, plan->partial, plan->counters,
                               reduce.data(), &plan->reduce_blocks);
    }
  }
  reduce.resize(rcount);
  plan->reduce_count = rcount;
  if (st == hipSuccess && tile == kGemmTile256x128) {
    map_wide_group_to_xcds(table.data(), count, blocks, &plan->block_map, &plan->reduce_map,
                           &plan->reduce_blocks);
    if (plan->block_map.help) {  // the GEMM launch sums its split tiles
      rcount = 0;
      reduce.clear();
      plan->reduce_count = 0;
    }
    if (count <= kInlineGroupMax) {
      GemmGroupLaunch& l = plan->wide_launch;
      l.tile = tile;
      l.w8 = w8;
      l.blocks = blocks;
      l.reducers = plan->reduce_blocks;
      for (int i = 0; i < count; ++i) l.g.d[i] = table[i];
      l.g.count = count;
      for (int i = 0; i < rcount; ++i) l.r.d[i] = reduce[i];
      l.r.count = rcount;
      l.gmap = plan->block_map;
      l.rmap = plan->reduce_map;
      plan->inline_wide = true;
    }
  }
  if (st == hipSuccess && !reduce.empty()) {
    st = hipMalloc(&plan->reduce, reduce.size() * sizeof(SplitReduceDesc));
    if (st == hipSuccess) {
      st = hipMemcpy(plan->reduce, reduce.data(), reduce.size() * sizeof(SplitReduceDesc),
                     hipMemcpyHostToDevice);
    }
  }
  if (st == hipSuccess) st = hipMalloc(&plan->table, table.size() * sizeof(GemmGroupDesc));
  if (st == hipSuccess) {
    st = hipMemcpy(plan->table, table.data(), table.size() * sizeof(GemmGroupDesc),
                   hipMemcpyHostToDevice);
  }
  if (st != hipSuccess) {
    if (plan->table) (void)hipFree(plan->table);
    if (plan->partial) (void)hipFree(plan->partial);
    if (plan->counters) (void)hipFree(plan->counters);
    if (plan->reduce) (void)hipFree(plan->reduce);
    delete plan;
    return fail(INFER_HIP_RUNTIME_ERROR, "gemm plan: %s", hipGetErrorString(st));
  }
  *plan_out = plan;
  return ok();
}

extern "C" int infer_hip_gemm_plan_launch(const infer_hip_gemm_plan* plan, hipStream_t stream) {
  if (!plan) return fail(INFER_HIP_INVALID_ARGUMENT, "gemm plan: null plan");
  if (plan->skinny) {
    launch_gemm_skinny(plan->w8, plan->skinny_args, plan->blocks, stream);
  } else if (plan->inline_wide) {
    launch_gemm_group_inline(plan->wide_launch, stream);
  } else if (plan->tile == kGemmTile256x128) {
    launch_gemm_wide_grouped(plan->w8, plan->table, plan->count, plan->blocks, plan->block_map,
                             plan->reduce, plan->reduce_count, plan->reduce_blocks,
                             plan->reduce_map, stream);
  } else {
    launch_gemm_grouped(plan->tile, plan->w8, plan->table, plan->count, plan->blocks, stream);
  }
  return check_launch("gemm plan");
}

extern "C" int infer_hip_gemm_plan_timeline(const infer_hip_gemm_plan* plan,
                                            unsigned long long* stamps, int capacity,
                                            int* workgroups, hipStream_t stream) {
  if (!plan || !workgroups) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "gemm plan timeline: null plan or output pointer");
  }
  if (plan->skinny || plan->tile != kGemmTile256x128) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "gemm plan timeline: only plans on the 256 x 128 tile (every GEMM with 256 "
                "tokens or more)");
  }
  *workgroups = plan->blocks;
  if (!stamps) return ok();
  if (capacity < plan->blocks) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "gemm plan timeline: stamps hold %d workgroups, the launch has %d", capacity,
                plan->blocks);
  }
  if (plan->inline_wide) {
    launch_gemm_wide_grouped_timeline(plan->wide_launch, stamps, stream);
  } else {
    launch_gemm_wide_grouped_timeline(plan->w8, plan->table, plan->count, plan->blocks,
                                      plan->block_map, stamps, plan->reduce, plan->reduce_count,
                                      plan->reduce_blocks, plan->reduce_map, stream);
  }
  return check_launch("gemm plan timeline");
}

extern "C" double infer_hip_gemm_plan_flops(const infer_hip_gemm_plan* plan) {
  return plan ? plan->flops : 0.0;
}

extern "C" int infer_hip_gemm_plan_destroy(infer_hip_gemm_plan* plan) {
  if (!plan) return ok();
  int prev = 0;
  hipError_t st = hipGetDevice(&prev);
  if (st == hipSuccess && prev != plan->device) st = hipSetDevice(plan->device);
  if (st == hipSuccess && plan->table) st = hipFree(plan->table);
  if (st == hipSuccess && plan->partial) st = hipFree(plan->partial);
  if (st == hipSuccess && plan->counters) st = hipFree(plan->counters);
  if (st == hipSuccess && plan->reduce) st = hipFree(plan->reduce);
  if (prev != plan->device) (void)hipSetDevice(prev);
  delete plan;
  if (st != hipSuccess) return fail(INFER_HIP_RUNTIME_ERROR, "gemm plan: %s", hipGetErrorString(st));
  return ok();
}
