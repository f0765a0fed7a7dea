// Internal launch interface between the kernel files (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace qlin {

struct W8GemvArgs {
  const int8_t* w;     // [n, k] int8
  const uint16_t* s;   // [n, k / 64] BF16 scales
  const uint16_t* bias;  // [n] BF16 or nullptr
  const uint16_t* x;   // [k] BF16
  uint16_t* y;         // [n] BF16
  int n;
  int k;
};

// One GEMV of a grouped launch; block_begin is the first block index of the
// launch that works on it (descriptors sorted by block_begin) and each of its
// blocks covers rows_per_block rows (a multiple of 4 waves x 8-row tasks).
struct W8GroupDesc {
  const int8_t* w;
  const uint16_t* s;
  const uint16_t* bias;
  const uint16_t* x;
  uint16_t* y;
  int n;
  int k;
  int block_begin;
  int rows_per_block;
};

struct Bf16GemvArgs {
  const uint16_t* w;     // [n, k] BF16
  const uint16_t* bias;  // [n] BF16 or nullptr
  const uint16_t* x;     // [k] BF16
  uint16_t* y;           // [n] BF16
  int n;
  int k;
};

// One GEMM Y[m, n] = bf16(sum_k X[m, k] W[n, k] + bias[n]); W is int8 with
// BF16 group-64 scales s (W8A16) or BF16 with s unused.
struct GemmArgs {
  const void* w;         // [n, k] int8 or BF16
  const uint16_t* s;     // [n, k / 64] BF16 scales (W8A16 only)
  const uint16_t* bias;  // [n] BF16 or nullptr
  const uint16_t* x;     // [m, k] BF16
  uint16_t* y;           // [m, n] BF16
  int m;
  int n;
  int k;
};

// Skinny GEMM for a few tokens (m <= kSkinnyMaxTokens): each workgroup
// streams 32 weight rows of one GEMM for 32 tokens, its waves splitting K
// (one workgroup per 32-token tile).  Up to
// kSkinnyMaxDescs GEMMs per launch (each on its own x and y), or one
// gate|up pair (w2, s2, bias2 set) writing bf16(silu(bf16(gate)) *
// bf16(up)).  block_begin is set by layout_skinny.  All GEMMs of a launch
// share m.
constexpr int kSkinnyMaxTokens = 128;
constexpr int kSkinnyMaxDescs = 8;
struct SkinnyDesc {
  const void* w;          // [n, k] int8 or BF16
  const uint16_t* s;      // [n, k / 64] BF16 scales (W8A16)
  const uint16_t* bias;   // [n] or nullptr
  const void* w2;         // pair: up_proj weight, else nullptr
  const uint16_t* s2;
  const uint16_t* bias2;
  const uint16_t* x;      // [m, k] BF16
  uint16_t* y;            // [m, n] BF16
  int n;
  int k;
  int block_begin;
  // K split over `parts` workgroups per 32-row block (layout_skinny): each
  // leaves a 32 x 32 FP32 partial in partial[(block * parts + part) *
  // 1024]; the last to arrive (counters[block], zero between launches)
  // sums them in part order.
  int parts;
  float* partial;
  int* counters;
};
struct SkinnyArgs {
  SkinnyDesc d[kSkinnyMaxDescs];
  int count;
  int m;
  int waves;  // per workgroup: 1, 2, 4 or 8 (layout_skinny)
};
bool gemm_skinny_supported(const void* w, const uint16_t* x, int m, int n, int k);
// Where the skinny kernel beats the 64 x 64 tiles (measured): up to 32
// tokens always, up to 64 on int8 weights; up to kSkinnyMaxTokens for
// narrow GEMMs (N <= 1024), on BF16 weights only up to 64 tokens unless K
// is long.  A token tile of 32 re-reads the weights, which wide GEMMs
// cannot afford.
bool gemm_skinny_preferred(bool w8, int m, int n, int k);
// Chooses the waves per workgroup and, with `split`, the K parts of long
// GEMMs (never of a pair); sets block_begin; returns the workgroup count.
// The split needs skinny_scratch() floats and counters, bound by
// bind_skinny().
int layout_skinny(SkinnyArgs& a, bool split);
void skinny_scratch(const SkinnyArgs& a, size_t* partial_floats, size_t* counters);
void bind_skinny(SkinnyArgs& a, float* partial, int* counters);
void launch_gemm_skinny(bool w8, const SkinnyArgs& a, int blocks, hipStream_t stream);

// MFMA GEMM workgroup tiles (rows x columns of Y).
enum GemmTile {
  kGemmTile128x128 = 0,
  kGemmTile128x64 = 1,
  kGemmTile64x128 = 2,
  kGemmTile64x64 = 3,
  kGemmTile32x128 = 4,
  kGemmTile256x128 = 5,  // 8 waves; grouped plans at M >= 256
  kGemmTileCount = 6,
};

// One GEMM of a grouped launch: its blocks are block_begin ..
// block_begin + tiles_m * tiles_n * splits - 1, each one part (of
// `splits`, split_stages K stages of 64 each) of one output tile of the
// plan's tile size (gemm_grouped_tile_rows x gemm_grouped_tile_cols).  Split tiles hand off through partial (splits FP32 tiles per
// output tile) and counters (one per output tile, zero between launches).
struct GemmGroupDesc {
  const void* w;
  const uint16_t* s;
  const uint16_t* bias;
  const uint16_t* x;
  uint16_t* y;
  int m;
  int n;
  int k;
  int tiles_m;
  int block_begin;
  int splits;
  int split_stages;
  float* partial;
  int* counters;
  // A gate|up pair (wide tile only, never split): w, s, bias are gate_proj,
  // w2, s2, bias2 up_proj, both [n / 2, k]; each 256 x 128 tile computes
  // 64 columns of both and writes y[:, 64 t ..] = bf16(silu(bf16(gate)) *
  // bf16(up)), y being [m, n / 2].  Null w2: a plain GEMM.
  const void* w2 = nullptr;
  const uint16_t* s2 = nullptr;
  const uint16_t* bias2 = nullptr;
  // The prefill's q|k|v epilogue (64 x 64 tiles, one head of 64 columns per
  // tile; rope_kind 0: the plain epilogue).  The tile's BF16 rows (bias
  // added, rounded) are, for kind 1, rotated by RoPE (pairs (i, i + 32),
  // the (cos, sin) of position rope_start + row at rope[position * 32 + i])
  // and written to y; kind 2, rotated and written to row rope_start + row of
  // kv_cache ([n / 64 heads][max_seq][64]); kind 3, written to kv_cache
  // unrotated.  Rows at or past max_seq are not written.
  const float2* rope = nullptr;
  uint16_t* kv_cache = nullptr;
  int rope_kind = 0;
  int rope_start = 0;
  int max_seq = 0;
};
// Split-K in the wide-tile grouped launch.  A GEMM whose wide tiles are
// split over K in `parts` parts writes each part's FP32 tile, row-major
// 256 x 128, to partial + (tile * parts + part) * 256 * 128 (tile = m_tile
// + tiles_m * n_tile); a second, reduction launch sums the parts in index
// order, adds the bias and writes BF16 Y.  Its blocks block_begin ..
// block_begin + tiles * 16 - 1 cover the GEMM, 16 rows of a tile each.
struct SplitReduceDesc {
  const float* partial;
  const uint16_t* bias;
  uint16_t* y;
  int m;
  int n;
  int tiles_m;
  int parts;
  int block_begin;
};
constexpr int kSplitReduceRows = 16;  // rows of a tile per reduction block

// XCD placement of a wide-tile plan.  Workgroup b of a launch runs on XCD
// b % 8, and each XCD has its own L2, so a split tile's parts are kept on one
// XCD and its reduction blocks on the same one: the FP32 parts are then
// written to and read back from that XCD's L2.  Both maps are permutations
// of the launches' logical blocks (any permutation gives the same results).
//
// Build options (measured alternatives, off by default; `make EXTRA_DEFS=...`):
// QLIN_WIDE_INKERNEL=1 sums a wide split tile's parts inside the GEMM launch
// (gemm.hip, wide_split_handoff) instead of in the reduction launch, with
// device-coherent (sc1) partial stores and loads, or with QLIN_HANDOFF_FENCE=1
// with plain accesses between agent-scope release and acquire fences, or
// with QLIN_HANDOFF_L2=1 (launches whose map keeps a tile's parts on one
// XCD) with plain accesses through that XCD's L2.
// QLIN_WIDE_DIRECT_A=1 (gemm.hip): the wide tile's X tiles go straight into
// LDS (buffer_load ... lds, two stages ahead into three swizzled buffers).
// QLIN_WIDE_HELP=1: on a mapped launch, every workgroup on an XCD that holds
// split tiles sums their slices once its own unit is done (gemm.hip,
// wide_split_help), so no reduction launch runs.
// QLIN_XCD_MAP=0 places workgroups in logical order.
// QLIN_GROUP_TILE128=1 (plan.cpp): a lone long-K GEMM of a `fill` group
// (K >= 2048, M >= 128: the prefill's down) on 128 x 128 tiles in 8 K parts
// instead of 64 x 64 tiles in up to 4 (measured at M = 512: 25.2 against
// 18.4 us per launch; at M = 128 within the run-to-run spread).
#ifndef QLIN_XCD_MAP
#define QLIN_XCD_MAP 1
#endif
#ifndef QLIN_WIDE_INKERNEL
#define QLIN_WIDE_INKERNEL 0
#endif
#ifndef QLIN_WIDE_HELP
#define QLIN_WIDE_HELP 0
#endif
// The in-launch hand-off: 4 ints of counters per split tile, at most 32 parts.
constexpr int kWideSplitCounterInts = 4;
constexpr int kWideMaxParts = 32;
constexpr int kXcds = 8;
constexpr int kWideMapBlocks = 256;  // plans with more blocks run unmapped
// The in-launch reduction by the XCD's workgroups: a 128-byte line of
// counters per split tile (arrived parts, next slice, departed workgroups),
// at most kHelpTiles split tiles per XCD.
constexpr int kHelpCounterInts = 32;
constexpr int kHelpTiles = 8;
struct WideBlockMap {
  int mapped = 0;                       // 0: workgroup b runs logical block b
  int help = 0;                         // 1: the launch sums its split tiles itself
  uint8_t logical[kWideMapBlocks] = {};  // workgroup -> logical block
  // help: split tiles (numbered over the launch's split descriptors in
  // order) whose parts run on XCD x, 0xFF: none
  uint8_t help_tiles[kXcds][kHelpTiles] = {};
  // help: workgroup -> its rank among the whole-tile workgroups of its XCD
  // (0xFF: a split part), and their number on each XCD
  uint8_t help_rank[kWideMapBlocks] = {};
  uint8_t help_members[kXcds] = {};
};
constexpr int kReduceSlots = 16;
struct ReduceBlockMap {
  // split tiles per XCD: the reduction launch has kXcds * slots *
  // (256 / kSplitReduceRows) workgroups; 0: unmapped
  int slots = 0;
  uint8_t tile[kXcds][kReduceSlots] = {};  // split tile of slot s on XCD x, 0xFF: none
};
// Places a wide-tile layout (after layout_gemm_group and bind_gemm_group) on
// the XCDs: each split tile's parts on the XCD with the most free workgroups,
// the whole tiles in the rest.  Leaves both maps unmapped when the launch has
// more than kWideMapBlocks blocks, no split tile, or a split tile that fits
// no XCD; *reducers receives the reduction launch's workgroups.
void map_wide_group_to_xcds(const GemmGroupDesc* descs, int count, int blocks, WideBlockMap* gmap,
                            ReduceBlockMap* rmap, int* reducers);

// A grouped launch laid out on the host and passed by value as kernel
// arguments, for callers whose shapes change from call to call (the model's
// prefill at the prompt's length): no descriptor table in device memory.
constexpr int kInlineGroupMax = 8;
struct GemmGroupArgs {
  GemmGroupDesc d[kInlineGroupMax];
  int count;
};
struct SplitReduceArgs {
  SplitReduceDesc d[kInlineGroupMax];
  int count;
};
struct GemmGroupLaunch {
  int tile;
  bool w8;
  int blocks;    // workgroups of the GEMM launch
  int reducers;  // workgroups of the split-K reduction launch (wide tile only)
  GemmGroupArgs g;
  SplitReduceArgs r;
  WideBlockMap gmap;   // wide tile: workgroup -> unit (map_wide_group_to_xcds)
  ReduceBlockMap rmap;
};

// plan.cpp: the layout shared by grouped plans and inline launches.  Sets
// every descriptor's tiles_m, splits, split_stages and block_begin (and
// sorts them, longest units first) for one launch on a device with `cus`
// CUs.  The tile is 256 x 128 once every GEMM has 256 rows or more (with
// `fill`, also only when the group has wide tiles for half the CUs), else
// 64 x 64.  K is split so that no unit is much longer than the group's
// shortest reduction (at least 8 stages), with parts lengthened until the
// units fit the device at once (one per CU on the wide tile, two on 64 x 64);
// with `fill`, for a lone or long-K group of one launch, into at most 4
// parts of at least 14 stages instead.
// Returns the tile; *blocks, *partial_floats and *counters receive the
// launch size and its split-K scratch needs.
int layout_gemm_group(GemmGroupDesc* descs, int count, int cus, bool fill, int* blocks,
                      size_t* partial_floats, size_t* counters);
// Points the split descriptors at `partial` / `counters` (sizes from
// layout_gemm_group) and writes the wide tile's reduction descriptors to
// reduce (at most count); returns the number of reduction descriptors and
// sets *reducers to the reduction launch's workgroups.
int bind_gemm_group(GemmGroupDesc* descs, int count, int tile, float* partial, int* counters,
                    SplitReduceDesc* reduce, int* reducers);
void launch_gemm_group_inline(const GemmGroupLaunch& l, hipStream_t stream);

// gemm.hip: gate_proj and up_proj of the same input, then SiLU-mul, as one
// launch of gate|up pair tiles (256 x 128 tiles, 64 columns of each; never
// split): y[m, n] = bf16(silu(bf16(x gate^T + gate_b)) * bf16(x up^T +
// up_b)), y [m, inter].  Supported when both GEMMs take the MFMA path.
bool gate_up_silu_supported(const void* gate_w, const void* up_w, const uint16_t* x, int m,
                            int inter, int hidden);
void launch_gate_up_silu(bool w8, const void* gate_w, const uint16_t* gate_s,
                         const uint16_t* gate_b, const void* up_w, const uint16_t* up_s,
                         const uint16_t* up_b, const uint16_t* x, uint16_t* y, int m, int inter,
                         int hidden, hipStream_t stream);

// The wide-tile grouped launch (`units` blocks over descs) and, when some
// GEMM is split, its reduction launch (`reducers` blocks over rdescs).
void launch_gemm_wide_grouped(bool w8, const GemmGroupDesc* descs, int count, int units,
                              const WideBlockMap& gmap, const SplitReduceDesc* rdescs, int rcount,
                              int reducers, const ReduceBlockMap& rmap, hipStream_t stream);
// The same, each workgroup of the GEMM launch writing 16 timeline words
// (entry, first stage, epilogue, end, XCD, hardware id, unit, shader cycles,
// and a split part's hand-off times) to stamps[16 b ..].
void launch_gemm_wide_grouped_timeline(bool w8, const GemmGroupDesc* descs, int count, int units,
                                       const WideBlockMap& gmap, unsigned long long* stamps,
                                       const SplitReduceDesc* rdescs, int rcount, int reducers,
                                       const ReduceBlockMap& rmap, hipStream_t stream);
// The same for launch_gemm_group_inline's wide-tile launches.
void launch_gemm_wide_grouped_timeline(const GemmGroupLaunch& l, unsigned long long* stamps,
                                       hipStream_t stream);

// gemm.hip
// Grouped launches use kGemmTile64x64, kGemmTile128x128 or kGemmTile256x128.
int gemm_tile_rows(int tile);
int gemm_tile_cols(int tile);
void launch_gemm_grouped(int tile, bool w8, const GemmGroupDesc* device_descs, int count,
                         int total_blocks, hipStream_t stream);
bool gemm_mfma_supported(const void* w, const uint16_t* x, int m, int n, int k);
int gemm_pick_tile(int m, int n);
void launch_gemm_mfma(int tile, bool w8, const GemmArgs& a, hipStream_t stream);

// gemv.hip
bool w8a16_gemv_fast_supported(const int8_t* w, const uint16_t* x, int k);
void launch_w8a16_gemv_fast(const W8GemvArgs& a, hipStream_t stream);
void launch_w8a16_linear_generic(const int8_t* w, const uint16_t* s, int group_size,
                                 const uint16_t* bias, const uint16_t* x, uint16_t* y,
                                 int tokens, int n, int k, hipStream_t stream);
bool bf16_gemv_fast_supported(const uint16_t* w, const uint16_t* x, int k);
void launch_bf16_gemv_fast(const Bf16GemvArgs& a, hipStream_t stream);
void launch_bf16_linear_generic(const uint16_t* w, const uint16_t* bias, const uint16_t* x,
                                uint16_t* y, int tokens, int n, int k, hipStream_t stream);
size_t lm_head_blocks(int vocab, int in_features, bool fast);

// Grouped W8A16 GEMV: rows per block for a descriptor of in_features k, and
// the launch of a descriptor table (any mix of K) resident on the device.
int w8a16_grouped_rows_per_block(int k);
void launch_w8a16_gemv_grouped(const W8GroupDesc* device_descs, int count, int total_blocks,
                               hipStream_t stream);

}  // namespace qlin
