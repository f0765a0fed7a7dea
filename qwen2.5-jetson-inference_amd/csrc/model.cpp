// Qwen2 decode runtime on the HIP Linear path: the device-side orchestration
// of Qwen2Model's BF16 / W8A16 prefill and decode (src/qwen2.cpp:496-743,
// Greedy-cy/qwen2.5-jetson-inference) behind the C ABI of infer_model.h.
//
// Memory: one device arena per model holds the decode state, the
// activations, the prefill workspace (max_sequence_length rows), the RoPE
// table, the attention partials, the grouped-GEMV descriptor tables and the
// KV cache; it is allocated once at creation, and no prefill or decode call
// allocates.
//
// Decode step (one token, position and token read from ModelState), W8A16
// or W16A16 (the same launches, on int8 or BF16 weights):
//   entry (the previous step's deferred argmax applied to the state, then
//   the token's embedding row); per layer five launches:
//     RMSNorm + q|k|v GEMV + RoPE + KV store (norm_qkv_rope),
//     attention over the context in kDecodeAttnParts parts (quarters:
//     one (acc, max, sum) record per head and part),
//     merge of the parts once per workgroup + o GEMV + residual
//     (attn_o_parts),
//     RMSNorm + gate|up GEMV + SiLU-mul (norm_gemv, paired rows),
//     down GEMV + residual (gemv_rows);
//   final RMSNorm + LM head + argmax (lm_head_decode, the argmax left in
//   lm_key for the next entry launch; a run of steps ends with one more
//   entry launch that only settles the state).
// Every launch is built to wait on one round of global loads: a decode
// step is latency-bound, not bandwidth-bound.  A head_dim other than 64 or
// a max_seq over 1024 changes only the attention and the o-projection: the
// split attention (RoPE applied inside it) and the span-merging o GEMV.  A
// hidden size beyond the fused kernels' limits (4096 with int8 weights,
// 2048 with BF16) runs unfused norm / GEMV / SiLU-mul launches around that
// split attention.  The down GEMV's residual add rides on the GEMV's bias operand
// (bias = output = the residual stream): each output element is read as
// bias and then written by the same lane, so the aliasing is safe.  With
// use_graph the step is captured once and replayed per token.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <initializer_list>
#include <new>
#include <string>
#include <vector>

#include "decode_kernels.hpp"
#include "infer_archive.h"
#include "infer_model.h"
#include "linear_kernels.hpp"
#include "model_kernels.hpp"
#include "status.hpp"

using namespace qlin;

namespace {

struct Linear {
  const void* w = nullptr;
  const uint16_t* s = nullptr;
  const uint16_t* b = nullptr;
  int n = 0;
  int k = 0;
};

struct Layer {
  const uint16_t* in_norm = nullptr;
  const uint16_t* post_norm = nullptr;
  Linear q, k, v, o, gate, up, down;
  uint16_t* key_cache = nullptr;
  uint16_t* value_cache = nullptr;
  // W8A16 grouped-GEMV descriptor tables (device) and their block counts
  // (the unfused path).
  W8GroupDesc* qkv_table = nullptr;
  W8GroupDesc* gate_up_table = nullptr;
  int qkv_blocks = 0;
  int gate_up_blocks = 0;
  // The fused path: RMSNorm + q|k|v, RMSNorm + gate|up + SiLU-mul.
  NormGemvArgs qkv_args{};
  QkvRopeArgs qkv_rope_args{};  // q|k|v + RoPE + KV store (whole-context attention)
  NormGemvArgs gate_up_args{};
  int qkv_fused_blocks = 0;
  int gate_up_fused_blocks = 0;
};

// Rows per block of the decode step's grouped GEMVs: one 4-row task per
// wave, the most blocks a grouped launch can have.
constexpr int kDecodeRowsPerBlock = 16;

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) & ~(kAlign - 1); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

double now_ms() {
  return std::chrono::duration<double, std::milli>(
             std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

}  // namespace

// Build option QLIN_PREFILL_GRAPH=1 (a measured alternative, off by
// default): with use_graph, a prompt length's prefill is captured as a graph
// the second time that length is prefilled and replayed from then on (a
// length seen once costs no capture).  Back-to-back kernels of a few us
// cost ~0.25 us less each in a graph than as stream launches, but the
// replayed Qwen2.5-0.5B prefill measured slower at 512 tokens (1.890 against
// 1.860 ms), 2 % faster at 128 and within the spread at 32.
#ifndef QLIN_PREFILL_GRAPH
#define QLIN_PREFILL_GRAPH 0
#endif
constexpr int kPrefillGraphs = 4;     // cached lengths (least recently used replaced)
constexpr int kPrefillSeen = 8;       // lengths remembered as prefilled once

struct PrefillGraph {
  int count = 0;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  unsigned long long used = 0;
};

struct infer_hip_model {
  infer_hip_model_config cfg{};
  bool w8 = false;
  bool use_graph = false;
  // hidden % 64 == 0, hidden <= 4096 (W8A16) or 2048 (W16A16)
  bool fused_norm_gemv = false;
  bool fused_lm_head = false;    // hidden % 8 == 0, hidden <= 4096
  // the fused q|k|v launch also rotates q, k and stores k, v (with the
  // whole-context decode attention: head_dim 64, max_seq <= 1024)
  bool fused_qkv_rope = false;
  int max_seq = 0;
  int head_dim = 0;
  int kv_dim = 0;
  int device = 0;
  hipStream_t stream = nullptr;
  char* arena = nullptr;
  size_t arena_bytes = 0;
  size_t kv_bytes = 0;
  int* pinned = nullptr;  // host readback slot (hipHostMalloc)
  void* owned_weights = nullptr;  // archive upload of infer_hip_model_open, else NULL

  ModelState* state = nullptr;
  int* history = nullptr;
  int* prompt = nullptr;
  uint16_t *x = nullptr, *norm = nullptr, *q = nullptr, *k = nullptr, *v = nullptr;
  uint16_t *gate = nullptr, *up = nullptr, *mlp = nullptr, *logits = nullptr;
  float* lm_value = nullptr;
  int* lm_index = nullptr;
  float* lm_best = nullptr;   // fused LM head: per-workgroup (value, index)
  int* lm_counter = nullptr;
  // fused LM head of the decode step: the argmax deferred to the next
  // step's entry launch (LmHeadDecodeArgs::key), zero when none is pending
  unsigned long long* lm_key = nullptr;
  float2* rope = nullptr;
  float2* rope_cur = nullptr;  // (cos, sin) of the decode position (RopeCursor)
  float* attn_partial = nullptr;  // decode attention split partials
  uint16_t* attn = nullptr;       // decode attention output (whole-context form)
  // split-K scratch of the prefill's grouped GEMM launches (sized at creation
  // for every prompt length up to max_seq)
  float* gemm_partial = nullptr;
  int* gemm_counters = nullptr;
  size_t gemm_partial_floats = 0;
  size_t gemm_counter_count = 0;
  int cus = 0;
  uint16_t *px = nullptr, *pnorm = nullptr, *pq = nullptr, *pk = nullptr, *pv = nullptr;
  uint16_t *pattn = nullptr, *ptmp = nullptr, *pgate = nullptr, *pup = nullptr, *pmlp = nullptr;

  const uint16_t* embed = nullptr;
  const uint16_t* final_norm = nullptr;
  const uint16_t* lm_head = nullptr;
  std::vector<Layer> layers;

  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  PrefillGraph prefill_graphs[kPrefillGraphs];
  int prefill_seen[kPrefillSeen] = {};
  int prefill_seen_next = 0;
  unsigned long long prefill_clock = 0;

  int position = 0;
  bool has_prefilled = false;
  int last_token = -1;
};

namespace qlin {

float2 rope_angle(float theta, int head_dim, int position, int i) {
  const float frequency = std::pow(theta, -2.0f * static_cast<float>(i) / head_dim);
  const float angle = static_cast<float>(position) * frequency;
  return make_float2(std::cos(angle), std::sin(angle));
}

}  // namespace qlin

namespace {

int hip_fail(hipError_t st, const char* what) {
  return fail(INFER_HIP_RUNTIME_ERROR, "%s: %s", what, hipGetErrorString(st));
}

// Makes the model's device current for the duration of a call.
class DeviceGuard {
 public:
  explicit DeviceGuard(int device) {
    if (hipGetDevice(&prev_) == hipSuccess && prev_ != device) {
      if (hipSetDevice(device) == hipSuccess) restore_ = true;
    }
  }
  ~DeviceGuard() {
    if (restore_) (void)hipSetDevice(prev_);
  }

 private:
  int prev_ = 0;
  bool restore_ = false;
};

// One token's GEMV (decode): W8A16 or BF16 fast path.
void gemv(const infer_hip_model* m, const Linear& l, const uint16_t* bias, const uint16_t* x,
          uint16_t* y) {
  if (m->w8) {
    launch_w8a16_gemv_fast({static_cast<const int8_t*>(l.w), l.s, bias, x, y, l.n, l.k},
                           m->stream);
  } else {
    launch_bf16_gemv_fast({static_cast<const uint16_t*>(l.w), bias, x, y, l.n, l.k}, m->stream);
  }
}

// token_count tokens (prefill): MFMA GEMM where it applies, the GEMV for
// one token, the exact generic kernel otherwise (src/qwen2.cpp:300-330).
void linear_batch(const infer_hip_model* m, const Linear& l, const uint16_t* x, uint16_t* y,
                  int tokens) {
  if (tokens == 1) {
    gemv(m, l, l.b, x, y);
  } else if (gemm_mfma_supported(l.w, x, tokens, l.n, l.k)) {
    launch_gemm_mfma(gemm_pick_tile(tokens, l.n), m->w8,
                     GemmArgs{l.w, l.s, l.b, x, y, tokens, l.n, l.k}, m->stream);
  } else if (m->w8) {
    launch_w8a16_linear_generic(static_cast<const int8_t*>(l.w), l.s, 64, l.b, x, y, tokens, l.n,
                                l.k, m->stream);
  } else {
    launch_bf16_linear_generic(static_cast<const uint16_t*>(l.w), l.b, x, y, tokens, l.n, l.k,
                               m->stream);
  }
}

// Several independent Linears of the prefill as one grouped MFMA launch
// (src/qwen2.cpp:300-330 per Linear), laid out for `tokens` rows with K split
// until the group covers the CUs; the split-K scratch is the arena's.  Falls
// back to one launch per Linear where the grouped kernels do not apply.
struct GemmItem {
  const Linear* l;
  const uint16_t* x;
  uint16_t* y;
};

// Up to kSkinnyMaxDescs Linears (or one gate|up pair with the SiLU-mul,
// pair_up set) as one skinny launch, for short prompts: the weights
// streamed once per 32 tokens, no tiles.  False where the skinny kernel does
// not apply or is not preferred (gemm_skinny_preferred).
bool skinny_group(const infer_hip_model* m, const GemmItem* items, int count, int tokens,
                  const Linear* pair_up = nullptr) {
  if (tokens < 2 || count > kSkinnyMaxDescs) return false;
  SkinnyArgs a{};
  a.count = count;
  a.m = tokens;
  for (int i = 0; i < count; ++i) {
    const Linear& l = *items[i].l;
    // An int8 gate|up pair takes the skinny pair launch up to
    // kSkinnyMaxTokens (beyond gemm_skinny_preferred's 64): it saves the
    // separate SiLU-mul launch (measured at Qwen2.5-0.5B shapes: TTFT 1.33-1.38
    // -> 1.27-1.28 ms at 96 tokens, 1.38-1.42 -> 1.37-1.38 at 128).
    const bool pair_w8 = pair_up && m->w8;
    if (!gemm_skinny_supported(l.w, items[i].x, tokens, l.n, l.k) ||
        !(pair_w8 || gemm_skinny_preferred(m->w8, tokens, pair_up ? 2 * l.n : l.n, l.k))) {
      return false;
    }
    a.d[i] = SkinnyDesc{l.w, m->w8 ? l.s : nullptr, l.b, nullptr, nullptr, nullptr,
                        items[i].x, items[i].y, l.n, l.k, 0};
  }
  if (pair_up) {
    if (count != 1 || pair_up->n != items[0].l->n || pair_up->k != items[0].l->k ||
        !gemm_skinny_supported(pair_up->w, items[0].x, tokens, pair_up->n, pair_up->k)) {
      return false;
    }
    a.d[0].w2 = pair_up->w;
    a.d[0].s2 = m->w8 ? pair_up->s : nullptr;
    a.d[0].bias2 = pair_up->b;
  }
  // K parts through the arena's split-K scratch (sized for them by
  // prefill_scratch_needs), shared with the tiled launches: one launch at
  // a time on the model's stream, and every counter back at zero after it.
  int blocks = layout_skinny(a, true);
  size_t pf = 0, cc = 0;
  skinny_scratch(a, &pf, &cc);
  if (pf <= m->gemm_partial_floats && cc <= m->gemm_counter_count) {
    bind_skinny(a, m->gemm_partial, m->gemm_counters);
  } else {
    blocks = layout_skinny(a, false);
  }
  launch_gemm_skinny(m->w8, a, blocks, m->stream);
  return true;
}

// The RoPE + KV store a q|k|v group can take into its epilogue (see
// GemmGroupDesc::rope_kind): items q, k, v in that order, head_dim 64.
struct QkvRope {
  const float2* table;
  uint16_t* key_cache;
  uint16_t* value_cache;
  int max_seq;
};

// Returns true when `rope` was given and the launch did the RoPE + KV store
// in its epilogue (the grouped launch on 64 x 64 tiles); otherwise the
// caller runs launch_rope_store.
bool linear_group(const infer_hip_model* m, const GemmItem* items, int count, int tokens,
                  const QkvRope* rope = nullptr) {
  if (skinny_group(m, items, count, tokens)) return false;
  bool grouped = tokens > 1 && count <= kInlineGroupMax;
  for (int i = 0; i < count && grouped; ++i) {
    grouped = gemm_mfma_supported(items[i].l->w, items[i].x, tokens, items[i].l->n,
                                  items[i].l->k);
  }
  GemmGroupLaunch g{};
  if (grouped) {
    for (int i = 0; i < count; ++i) {
      const Linear& l = *items[i].l;
      g.g.d[i] = GemmGroupDesc{l.w, m->w8 ? l.s : nullptr, l.b, items[i].x, items[i].y, tokens,
                               l.n, l.k, 0, 0, 1, l.k / 64, nullptr, nullptr};
    }
    g.g.count = count;
    g.w8 = m->w8;
    if (rope && count == 3) {  // set before the layout, which reorders the descriptors
      for (int i = 0; i < 3; ++i) {
        GemmGroupDesc& d = g.g.d[i];
        d.rope = rope->table;
        d.rope_kind = i + 1;  // q rotated in place, k rotated into its cache, v into its cache
        d.kv_cache = i == 1 ? rope->key_cache : (i == 2 ? rope->value_cache : nullptr);
        d.rope_start = 0;
        d.max_seq = rope->max_seq;
      }
    }
    size_t pf = 0, cc = 0;
    g.tile = layout_gemm_group(g.g.d, count, m->cus, true, &g.blocks, &pf, &cc);
    grouped = g.blocks > 0 && pf <= m->gemm_partial_floats && cc <= m->gemm_counter_count;
  }
  if (!grouped) {
    for (int i = 0; i < count; ++i) linear_batch(m, *items[i].l, items[i].x, items[i].y, tokens);
    return false;
  }
  g.r.count = bind_gemm_group(g.g.d, count, g.tile, m->gemm_partial, m->gemm_counters, g.r.d,
                              &g.reducers);
  if (g.tile == kGemmTile256x128) {
    map_wide_group_to_xcds(g.g.d, count, g.blocks, &g.gmap, &g.rmap, &g.reducers);
    if (g.gmap.help) g.r.count = 0;  // the GEMM launch sums its split tiles
  }
  launch_gemm_group_inline(g, m->stream);
  return rope && count == 3 && g.tile == kGemmTile64x64;
}

// gate|up + SiLU-mul of the prefill as one launch of pair tiles: where the
// two GEMMs' own grouped launch would take the wide tile unsplit (prompts
// over 256 tokens at the Qwen2.5-0.5B shapes), so the same tiles also
// write the SiLU-mul instead of two BF16 outputs and a third launch.
bool fuse_gate_up(const infer_hip_model* m, const Layer& L, int tokens) {
  if (!gate_up_silu_supported(L.gate.w, L.up.w, m->pnorm, tokens, L.gate.n, L.gate.k)) {
    return false;
  }
  GemmGroupDesc d[2] = {
      {L.gate.w, L.gate.s, L.gate.b, m->pnorm, m->pgate, tokens, L.gate.n, L.gate.k, 0, 0, 1,
       L.gate.k / 64, nullptr, nullptr},
      {L.up.w, L.up.s, L.up.b, m->pnorm, m->pup, tokens, L.up.n, L.up.k, 0, 0, 1, L.up.k / 64,
       nullptr, nullptr}};
  int blocks = 0;
  size_t pf = 0, cc = 0;
  const int tile = layout_gemm_group(d, 2, m->cus, true, &blocks, &pf, &cc);
  return tile == kGemmTile256x128 && d[0].splits == 1 && d[1].splits == 1;
}

// The split-K scratch the prefill's groups (q|k|v, o, gate|up, down) need at
// any prompt length up to max_seq.
void prefill_scratch_needs(const infer_hip_model_config& c, int head_dim, int max_seq, int cus,
                           size_t* partial_floats, size_t* counters) {
  const int hidden = c.hidden_size, inter = c.intermediate_size;
  const int kv_dim = c.num_kv_heads * head_dim;
  const int shapes[4][3][2] = {{{hidden, hidden}, {kv_dim, hidden}, {kv_dim, hidden}},
                               {{hidden, hidden}, {0, 0}, {0, 0}},
                               {{inter, hidden}, {inter, hidden}, {0, 0}},
                               {{hidden, inter}, {0, 0}, {0, 0}}};
  const int counts[4] = {3, 1, 2, 1};
  *partial_floats = 0;
  *counters = 0;
  for (int tokens = 2; tokens <= max_seq; ++tokens) {
    for (int g = 0; g < 4; ++g) {
      GemmGroupDesc d[kInlineGroupMax] = {};
      for (int i = 0; i < counts[g]; ++i) {
        d[i].m = tokens;
        d[i].n = shapes[g][i][0];
        d[i].k = shapes[g][i][1];
      }
      int blocks = 0;
      size_t pf = 0, cc = 0;
      (void)layout_gemm_group(d, counts[g], cus, true, &blocks, &pf, &cc);
      *partial_floats = std::max(*partial_floats, pf);
      *counters = std::max(*counters, cc);
    }
  }
  // The skinny launches' K parts (prompts of 2 .. kSkinnyMaxTokens tokens;
  // the most at the most tokens: one tile of parts per 32 tokens).
  for (int g = 0; g < 4; ++g) {
    SkinnyArgs a{};
    a.count = counts[g];
    a.m = std::min(max_seq, kSkinnyMaxTokens);
    for (int i = 0; i < counts[g]; ++i) {
      a.d[i].n = shapes[g][i][0];
      a.d[i].k = shapes[g][i][1];
    }
    (void)layout_skinny(a, true);
    size_t pf = 0, cc = 0;
    skinny_scratch(a, &pf, &cc);
    *partial_floats = std::max(*partial_floats, pf);
    *counters = std::max(*counters, cc);
  }
}

// The model's RoPE cursor: its table and the row of the decode position.
RopeCursor rope_cursor(const infer_hip_model* m) {
  return RopeCursor{m->rope, m->rope_cur, m->head_dim / 2, m->max_seq};
}

// Final RMSNorm of `row` and the LM head with its argmax into state->token;
// with `advance` the step's bookkeeping too (history, step, position).  The
// fused LM head of a decode step defers both: its argmax stays in m->lm_key
// for the next decode_entry launch (enqueue_decode_step, finish_decode).
// add (optional): the row normalized is bf16(row + add), the residual add
// the prefill's last layer leaves for the one row read here (the unfused
// path writes it into the row first).
int lm_head_step(infer_hip_model* m, const uint16_t* row, bool advance, bool defer = false,
                 const uint16_t* add = nullptr) {
  const infer_hip_model_config& c = m->cfg;
  if (m->fused_lm_head) {
    LmHeadDecodeArgs a{row, m->final_norm, c.rms_norm_eps, m->lm_head, c.vocab_size,
                       c.hidden_size, m->logits, m->lm_best, m->lm_counter,
                       &m->state->token, m->state, m->history, m->max_seq,
                       defer ? 2 : (advance ? 1 : 0), rope_cursor(m)};
    a.key = m->lm_key;
    a.x_add = add;
    launch_lm_head_decode(a, m->stream);
    return check_launch("lm head");
  }
  if (add) launch_add(const_cast<uint16_t*>(row), add, c.hidden_size, m->stream);
  launch_rms_norm(row, m->final_norm, m->norm, 1, c.hidden_size, c.rms_norm_eps, m->stream);
  const int rc = infer_hip_lm_head_bf16(m->lm_head, nullptr, m->norm, m->logits, m->lm_value,
                                        m->lm_index, &m->state->token, c.vocab_size,
                                        c.hidden_size, m->stream);
  if (rc != INFER_HIP_OK || !advance) return rc;
  launch_advance(m->state, m->history, m->max_seq, rope_cursor(m), m->stream);
  return check_launch("decode step advance");
}

// The entry launch of a decode step (and, with out null, the launch that
// applies the last step's deferred argmax: finish_decode).
DecodeEntryArgs entry_args(const infer_hip_model* m, uint16_t* out) {
  return DecodeEntryArgs{m->embed, m->state, m->lm_key, m->history, m->max_seq,
                         rope_cursor(m), m->cfg.vocab_size, m->cfg.hidden_size, out};
}

// After the last decode step of a run: the step's deferred argmax applied
// to the state (token, history, step, position, RoPE row).
int finish_decode(infer_hip_model* m) {
  if (!m->fused_lm_head) return ok();
  launch_decode_entry(entry_args(m, nullptr), m->stream);
  return check_launch("decode finish");
}

// Launch kinds of a decode step, for infer_hip_model_kernel_times.
enum StepKind {
  kKindEmbedding = 0,
  kKindNorm,       // RMSNorm (unfused paths)
  kKindQkv,        // q|k|v GEMV(s) (W8A16: with the RMSNorm)
  kKindAttention,  // RoPE + KV store + split attention
  kKindAttnO,      // split merge + o GEMV + residual
  kKindGateUp,     // gate|up GEMV(s) (W8A16: with the RMSNorm and SiLU-mul)
  kKindSiluMul,    // SiLU-mul (unfused paths)
  kKindDown,       // down GEMV + residual
  kKindLmHead,     // final RMSNorm + LM head + argmax + step bookkeeping
  kKindCount
};

const char* const kKindNames[kKindCount] = {
    "embedding", "rms_norm", "qkv_gemv", "attention", "attn_o_gemv",
    "gate_up_gemv", "silu_mul", "down_gemv", "lm_head"};

// Enqueue one decode step (src/qwen2.cpp:597-674) on the model's stream.
// only >= 0 enqueues just the launches of that kind; events (only with
// `only`) gets one record before the first launch and one after each.
int enqueue_decode_step(infer_hip_model* m, int only = -1, hipEvent_t* events = nullptr) {
  const infer_hip_model_config& c = m->cfg;
  const int hidden = c.hidden_size;
  hipStream_t s = m->stream;
  int recorded = 0;
  if (events) (void)hipEventRecord(events[recorded++], s);
  auto run = [&](int kind, auto&& launch) {
    if (only >= 0 && only != kind) return;
    launch();
    if (events) (void)hipEventRecord(events[recorded++], s);
  };
  run(kKindEmbedding, [&] {
    if (m->fused_lm_head) {
      launch_decode_entry(entry_args(m, m->x), s);
    } else {
      launch_embedding(m->embed, &m->state->token, 1, c.vocab_size, hidden, m->x, s);
    }
  });
  for (const Layer& L : m->layers) {
    if (m->fused_norm_gemv) {
      if (m->fused_qkv_rope) {
        run(kKindQkv, [&] { launch_norm_qkv_rope(L.qkv_rope_args, m->w8, s); });
      } else {
        run(kKindQkv,
            [&] { launch_norm_gemv(L.qkv_args, L.qkv_fused_blocks, false, m->w8, s); });
      }
    } else {
      run(kKindNorm,
          [&] { launch_rms_norm(m->x, L.in_norm, m->norm, 1, hidden, c.rms_norm_eps, s); });
      if (m->w8) {
        run(kKindQkv, [&] { launch_w8a16_gemv_grouped(L.qkv_table, 3, L.qkv_blocks, s); });
      } else {
        run(kKindQkv, [&] { gemv(m, L.q, L.q.b, m->norm, m->q); });
        run(kKindQkv, [&] { gemv(m, L.k, L.k.b, m->norm, m->k); });
        run(kKindQkv, [&] { gemv(m, L.v, L.v.b, m->norm, m->v); });
      }
    }
    run(kKindAttention, [&] {
      if (m->fused_qkv_rope) {
        launch_attention_decode_parts(m->q, L.key_cache, L.value_cache, &m->state->pos,
                                      c.num_heads, c.num_kv_heads, m->max_seq,
                                      m->attn_partial, s, kDecodeAttnParts);
      } else {
        launch_attention_decode(m->q, m->k, m->v, L.key_cache, L.value_cache, m->rope,
                                &m->state->pos, c.num_heads, c.num_kv_heads, m->head_dim,
                                m->max_seq, false, m->attn_partial, m->attn, s);
      }
    });
    // x = bf16(Wo attn + x): attn is merged here from the attention's
    // partials (the kDecodeAttnParts parts, or the spans of the split form)
    run(kKindAttnO, [&] {
      if (m->fused_qkv_rope) {
        launch_attn_o_parts({m->attn_partial, &m->state->pos, c.num_heads, m->max_seq, L.o.w,
                             L.o.s, m->x, hidden, hidden},
                            m->w8, s, kDecodeAttnParts);
      } else {
        launch_attn_o_gemv({m->attn_partial, &m->state->pos, c.num_heads, m->head_dim,
                            attention_span(m->max_seq, m->head_dim),
                            attention_splits(m->max_seq, m->head_dim), m->max_seq, L.o.w, L.o.s,
                            m->x, hidden, hidden},
                           m->w8, s);
      }
    });
    if (m->fused_norm_gemv) {
      run(kKindGateUp,
          [&] { launch_norm_gemv(L.gate_up_args, L.gate_up_fused_blocks, true, m->w8, s); });
    } else {
      run(kKindNorm,
          [&] { launch_rms_norm(m->x, L.post_norm, m->norm, 1, hidden, c.rms_norm_eps, s); });
      if (m->w8) {
        run(kKindGateUp,
            [&] { launch_w8a16_gemv_grouped(L.gate_up_table, 2, L.gate_up_blocks, s); });
      } else {
        run(kKindGateUp, [&] { gemv(m, L.gate, nullptr, m->norm, m->gate); });
        run(kKindGateUp, [&] { gemv(m, L.up, nullptr, m->norm, m->up); });
      }
      run(kKindSiluMul,
          [&] { launch_silu_mul(m->gate, m->up, m->mlp, c.intermediate_size, s); });
    }
    run(kKindDown, [&] {  // x = bf16(Wd mlp + x)
      if (gemv_rows_supported(L.down.k, m->w8)) {
        launch_gemv_rows({L.down.w, L.down.s, m->x, m->mlp, m->x, L.down.n, L.down.k}, m->w8,
                         s);
      } else {
        gemv(m, L.down, m->x, m->mlp, m->x);
      }
    });
  }
  int rc = check_launch("decode step");
  if (rc != INFER_HIP_OK) return rc;
  run(kKindLmHead, [&] { rc = lm_head_step(m, m->x, only < 0, true); });
  return rc;
}

// Compulsory HBM bytes of one decode step's launches of `kind` at context
// length ctx (positions [0, ctx)), and how many launches the step has.
double kind_bytes(const infer_hip_model* m, int kind, int ctx, int* launches) {
  const infer_hip_model_config& c = m->cfg;
  const double H = c.hidden_size, I = c.intermediate_size, V = c.vocab_size;
  const double KV = m->kv_dim, hd = m->head_dim, nl = c.num_layers;
  const double wb = m->w8 ? 1.0 : 2.0;  // weight bytes per element
  auto linear = [&](double n, double k) {
    return n * k * wb + (m->w8 ? 2.0 * n * (k / 64) : 0.0);
  };
  // the attention's output: the (acc, max, sum) records of the parts or
  // of the split form's spans (a record's padding is not counted)
  const int span = m->fused_qkv_rope ? kAttnWholeMax / kDecodeAttnParts
                                     : attention_span(m->max_seq, m->head_dim);
  const double splits = (ctx + span - 1) / span;
  const double partials = c.num_heads * splits * (hd + 2) * 4;
  const bool fused = m->fused_norm_gemv;
  const bool bf16_split = !m->w8 && !fused;  // separate q, k, v (and gate, up) launches
  int n = 0;
  double b = 0.0;
  switch (kind) {
    case kKindEmbedding:
      n = 1;
      b = 4 * H;
      break;
    case kKindNorm:
      n = fused ? 0 : 2 * c.num_layers;
      b = n * 6 * H;
      break;
    case kKindQkv:
      n = c.num_layers * (bf16_split ? 3 : 1);
      b = nl * (linear(H + 2 * KV, H) + 2 * (H + 2 * KV) /* bias */ +
                2 * (H + 2 * KV) /* out */ + (fused ? 4 * H : 2 * H * (bf16_split ? 3 : 1)));
      break;
    case kKindAttention:
      n = c.num_layers;
      b = m->fused_qkv_rope
              ? nl * (2 * c.num_kv_heads * ctx * hd * 2 /* K, V rows, the new one included */ +
                      2 * H /* q */ + partials)
              : nl * (2 * c.num_kv_heads * (ctx - 1) * hd * 2 /* cached K, V */ +
                      2 * H /* q */ + 4 * KV /* new k, v */ + 4 * KV /* their store */ +
                      partials);
      break;
    case kKindAttnO:
      n = c.num_layers;
      b = nl * (linear(H, H) + partials + 4 * H);
      break;
    case kKindGateUp:
      n = c.num_layers * (bf16_split ? 2 : 1);
      b = nl * (2 * linear(I, H) +
                (fused ? 4 * H + 2 * I : 2 * H * (bf16_split ? 2 : 1) + 4 * I));
      break;
    case kKindSiluMul:
      n = fused ? 0 : c.num_layers;
      b = n * 6 * I;
      break;
    case kKindDown:
      n = c.num_layers;
      b = nl * (linear(H, I) + 2 * I + 4 * H);
      break;
    case kKindLmHead:
      n = 1;
      b = V * H * 2 + 4 * H + 2 * V;
      break;
    default:
      break;
  }
  *launches = n;
  return b;
}

int ensure_graph(infer_hip_model* m) {
  if (m->graph_exec) return ok();
  hipError_t st = hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal);
  if (st != hipSuccess) return hip_fail(st, "decode graph capture");
  const int rc = enqueue_decode_step(m);
  hipGraph_t graph = nullptr;
  st = hipStreamEndCapture(m->stream, &graph);
  if (rc != INFER_HIP_OK) {
    if (graph) (void)hipGraphDestroy(graph);
    return rc;
  }
  if (st != hipSuccess) return hip_fail(st, "decode graph capture");
  hipGraphExec_t exec = nullptr;
  st = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (st != hipSuccess) {
    (void)hipGraphDestroy(graph);
    return hip_fail(st, "decode graph instantiate");
  }
  m->graph = graph;
  m->graph_exec = exec;
  return ok();
}

int run_decode_step(infer_hip_model* m) {
  if (m->use_graph) {
    const hipError_t st = hipGraphLaunch(m->graph_exec, m->stream);
    return st == hipSuccess ? ok() : hip_fail(st, "decode graph launch");
  }
  return enqueue_decode_step(m);
}

int read_token(infer_hip_model* m, int* out) {
  hipError_t st = hipMemcpyAsync(m->pinned, &m->state->token, sizeof(int),
                                 hipMemcpyDeviceToHost, m->stream);
  if (st == hipSuccess) st = hipStreamSynchronize(m->stream);
  if (st != hipSuccess) return hip_fail(st, "token readback");
  *out = *m->pinned;
  return ok();
}

int enqueue_prefill(infer_hip_model* m, int count);
hipGraphExec_t prefill_graph(infer_hip_model* m, int count);

// src/qwen2.cpp:496-595 on the model's stream; returns the argmax.
int run_prefill(infer_hip_model* m, const int* tokens, int count, int* next) {
  hipStream_t s = m->stream;
  if (count == 1) {
    // A one-token prompt is the decode step at position 0 (one graph
    // replay, 5 launches per layer) rather than the M = 1 prefill (9 per
    // layer): 0.5 ms instead of 1.0 ms for Qwen2.5-0.5B.
    launch_set_state(m->state, tokens[0], 0, 0, rope_cursor(m), s, m->lm_key);
    int rc = check_launch("prefill state");
    if (rc == INFER_HIP_OK) rc = run_decode_step(m);
    if (rc == INFER_HIP_OK) rc = finish_decode(m);
    if (rc == INFER_HIP_OK) rc = read_token(m, next);
    return rc;
  }
  hipError_t st = hipMemcpyAsync(m->prompt, tokens, sizeof(int) * count, hipMemcpyHostToDevice, s);
  if (st != hipSuccess) return hip_fail(st, "prefill token upload");
  const hipGraphExec_t exec =
      QLIN_PREFILL_GRAPH && m->use_graph ? prefill_graph(m, count) : nullptr;
  int rc = INFER_HIP_OK;
  if (exec) {
    st = hipGraphLaunch(exec, s);
    if (st != hipSuccess) return hip_fail(st, "prefill graph launch");
  } else {
    rc = enqueue_prefill(m, count);
  }
  if (rc != INFER_HIP_OK) return rc;
  return read_token(m, next);
}

// The prefill's launches for a `count`-token prompt already in m->prompt,
// through the state update (its argmax in state->token).
int enqueue_prefill(infer_hip_model* m, int count) {
  const infer_hip_model_config& c = m->cfg;
  const int hidden = c.hidden_size, inter = c.intermediate_size;
  hipStream_t s = m->stream;
  launch_embedding_rms_norm(m->embed, m->prompt, count, c.vocab_size, hidden, m->px,
                            m->layers[0].in_norm, m->pnorm, c.rms_norm_eps, s);
  // The residual adds ride with the RMSNorm behind them (after o: the
  // post-attention norm; after down: the next layer's input norm).
  for (size_t l = 0; l < m->layers.size(); ++l) {
    const Layer& L = m->layers[l];
    const GemmItem qkv[3] = {{&L.q, m->pnorm, m->pq}, {&L.k, m->pnorm, m->pk},
                             {&L.v, m->pnorm, m->pv}};
    // RoPE + KV store in the q|k|v launch's epilogue where its tiles hold
    // whole heads (64 x 64 tiles, head_dim 64), else their own launch
    const QkvRope rope{m->rope, L.key_cache, L.value_cache, m->max_seq};
    // (short prompts, whose q|k|v runs on the skinny kernel: inside the
    // attention launch instead)
    if (linear_group(m, qkv, 3, count, m->head_dim == 64 ? &rope : nullptr)) {
      launch_attention_prefill(m->pq, L.key_cache, L.value_cache, m->pattn, count,
                               c.num_heads, c.num_kv_heads, m->head_dim, m->max_seq, s);
    } else if (!attention_prefill_rope(m->pq, m->pk, m->pv, L.key_cache, L.value_cache,
                                       m->rope, m->pattn, count, c.num_heads, c.num_kv_heads,
                                       m->head_dim, m->max_seq, s)) {
      launch_rope_store(m->pq, m->pk, m->pv, L.key_cache, L.value_cache, m->rope, count, 0,
                        c.num_heads, c.num_kv_heads, m->head_dim, m->max_seq, s);
      launch_attention_prefill(m->pq, L.key_cache, L.value_cache, m->pattn, count,
                               c.num_heads, c.num_kv_heads, m->head_dim, m->max_seq, s);
    }
    const GemmItem o[1] = {{&L.o, m->pattn, m->ptmp}};
    linear_group(m, o, 1, count);
    launch_add_rms_norm(m->px, m->ptmp, L.post_norm, m->pnorm, count, hidden, c.rms_norm_eps, s);
    const GemmItem gate_silu[1] = {{&L.gate, m->pnorm, m->pmlp}};
    if (fuse_gate_up(m, L, count)) {
      launch_gate_up_silu(m->w8, L.gate.w, L.gate.s, L.gate.b, L.up.w, L.up.s, L.up.b, m->pnorm,
                          m->pmlp, count, inter, hidden, s);
    } else if (skinny_group(m, gate_silu, 1, count, &L.up)) {
      // gate|up + SiLU-mul as one skinny pair launch
    } else {
      const GemmItem gate_up[2] = {{&L.gate, m->pnorm, m->pgate}, {&L.up, m->pnorm, m->pup}};
      linear_group(m, gate_up, 2, count);
      launch_silu_mul(m->pgate, m->pup, m->pmlp, static_cast<long long>(count) * inter, s);
    }
    const GemmItem down[1] = {{&L.down, m->pmlp, m->ptmp}};
    linear_group(m, down, 1, count);
    // the last layer's residual add is needed for the last row only: the
    // LM head step takes it
    if (l + 1 < m->layers.size()) {
      launch_add_rms_norm(m->px, m->ptmp, m->layers[l + 1].in_norm, m->pnorm, count, hidden,
                          c.rms_norm_eps, s);
    }
  }
  int rc = check_launch("prefill");
  if (rc != INFER_HIP_OK) return rc;
  const size_t last = static_cast<size_t>(count - 1) * hidden;
  rc = lm_head_step(m, m->px + last, false, false, m->ptmp + last);
  if (rc != INFER_HIP_OK) return rc;
  launch_set_state(m->state, -1, count, 0, rope_cursor(m), s, m->lm_key);
  return check_launch("prefill state");
}

// The cached graph of a `count`-token prefill (captured here on the
// length's second prefill), or null: run the launches directly.  A capture
// that fails leaves nothing behind and the prefill runs directly.
hipGraphExec_t prefill_graph(infer_hip_model* m, int count) {
  for (PrefillGraph& g : m->prefill_graphs) {
    if (g.exec && g.count == count) {
      g.used = ++m->prefill_clock;
      return g.exec;
    }
  }
  bool seen = false;
  for (int v : m->prefill_seen) seen = seen || v == count;
  if (!seen) {
    m->prefill_seen[m->prefill_seen_next] = count;
    m->prefill_seen_next = (m->prefill_seen_next + 1) % kPrefillSeen;
    return nullptr;
  }
  if (hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  const int rc = enqueue_prefill(m, count);
  hipGraph_t graph = nullptr;
  hipError_t st = hipStreamEndCapture(m->stream, &graph);
  hipGraphExec_t exec = nullptr;
  if (rc == INFER_HIP_OK && st == hipSuccess && graph) {
    st = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  }
  if (rc != INFER_HIP_OK || st != hipSuccess || !exec) {
    if (graph) (void)hipGraphDestroy(graph);
    (void)hipGetLastError();
    return nullptr;
  }
  PrefillGraph* slot = &m->prefill_graphs[0];
  for (PrefillGraph& g : m->prefill_graphs) {
    if (!g.exec) {
      slot = &g;
      break;
    }
    if (g.used < slot->used) slot = &g;
  }
  if (slot->exec) (void)hipGraphExecDestroy(slot->exec);
  if (slot->graph) (void)hipGraphDestroy(slot->graph);
  *slot = PrefillGraph{count, graph, exec, ++m->prefill_clock};
  return exec;
}

int check_linear(const infer_hip_linear& l, bool w8, bool want_bias, int n, int k, int layer,
                 const char* name) {
  if (!l.weight || (w8 && !l.scales)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model: layer %d %s: null weight or scales", layer,
                name);
  }
  if (!want_bias && l.bias) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model: layer %d %s takes no bias", layer, name);
  }
  // The fast GEMV paths: K a multiple of 64 (W8A16) or 8 (BF16), 16-byte
  // aligned weight (activations are arena buffers, 256-byte aligned).
  const int k_align = w8 ? 64 : 8;
  const bool fast = k >= k_align && k % k_align == 0 && aligned16(l.weight);
  if (!fast || (l.bias && !aligned16(l.bias)) || (l.scales && !aligned16(l.scales))) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "model: layer %d %s [%d, %d]: needs 16-byte aligned tensors and in_features %% "
                "%d == 0",
                layer, name, n, k, k_align);
  }
  return ok();
}

void destroy_model(infer_hip_model* m) {
  if (!m) return;
  DeviceGuard guard(m->device);
  if (m->stream) (void)hipStreamSynchronize(m->stream);
  if (m->graph_exec) (void)hipGraphExecDestroy(m->graph_exec);
  if (m->graph) (void)hipGraphDestroy(m->graph);
  for (PrefillGraph& g : m->prefill_graphs) {
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
    if (g.graph) (void)hipGraphDestroy(g.graph);
  }
  if (m->arena) (void)hipFree(m->arena);
  if (m->owned_weights) (void)hipFree(m->owned_weights);
  if (m->pinned) (void)hipHostFree(m->pinned);
  if (m->stream) (void)hipStreamDestroy(m->stream);
  delete m;
}

}  // namespace

extern "C" int infer_hip_model_create(const infer_hip_model_config* config,
                                      const infer_hip_model_weights* weights,
                                      const infer_hip_runtime_options* options,
                                      infer_hip_model** out) {
  if (!out) return fail(INFER_HIP_INVALID_ARGUMENT, "model: null output pointer");
  *out = nullptr;
  if (!config || !weights || !options || !weights->layers) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model: null config, weights or options");
  }
  const infer_hip_model_config& c = *config;
  // model_config.cpp:42-48 plus what the HIP kernels need.
  if (c.hidden_size <= 0 || c.intermediate_size <= 0 || c.num_layers <= 0 || c.vocab_size <= 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model: invalid model dimensions");
  }
  if (c.num_heads <= 0 || c.num_kv_heads <= 0 || c.num_heads % c.num_kv_heads != 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model: invalid GQA head counts");
  }
  if (c.hidden_size % c.num_heads != 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model: invalid attention head dimension");
  }
  const int head_dim = c.hidden_size / c.num_heads;
  if (!attention_head_dim_supported(head_dim)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model: head_dim %d unsupported (64 or 128)",
                head_dim);
  }
  if (!attn_o_supported(c.hidden_size, c.num_heads, options->precision == INFER_HIP_PRECISION_W8A16) ||
      c.num_heads > kAttnOMaxHeads) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "model: %d attention heads / hidden %d unsupported by the decode attention "
                "(at most %d heads, hidden <= 4096)",
                c.num_heads, c.hidden_size, kAttnOMaxHeads);
  }
  if (!(c.rms_norm_eps >= 0.0f) || !(c.rope_theta > 0.0f)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model: invalid rms_norm_eps or rope_theta");
  }
  const int precision = options->precision;
  if (precision != INFER_HIP_PRECISION_W16A16 && precision != INFER_HIP_PRECISION_W8A16) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "model: precision must be W16A16 or W8A16 (the FP32 path is the CPU's)");
  }
  const int max_seq = options->max_sequence_length;
  if (max_seq <= 0) return fail(INFER_HIP_INVALID_ARGUMENT, "model: max_sequence_length <= 0");
  const bool w8 = precision == INFER_HIP_PRECISION_W8A16;
  const int hidden = c.hidden_size, inter = c.intermediate_size;
  const int kv_dim = c.num_kv_heads * head_dim;

  if (!weights->embed_tokens || !weights->norm) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model: null embedding or final norm");
  }
  const uint16_t* lm_head = weights->lm_head ? weights->lm_head : weights->embed_tokens;
  if (!aligned16(lm_head) || !aligned16(weights->embed_tokens) || hidden % 8 != 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "model: embedding / LM head need 16-byte alignment and hidden %% 8 == 0");
  }
  for (int l = 0; l < c.num_layers; ++l) {
    const infer_hip_layer_weights& L = weights->layers[l];
    if (!L.input_layernorm || !L.post_attention_layernorm) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "model: layer %d: null norm weight", l);
    }
    int rc = check_linear(L.q_proj, w8, true, hidden, hidden, l, "q_proj");
    if (rc == INFER_HIP_OK) rc = check_linear(L.k_proj, w8, true, kv_dim, hidden, l, "k_proj");
    if (rc == INFER_HIP_OK) rc = check_linear(L.v_proj, w8, true, kv_dim, hidden, l, "v_proj");
    if (rc == INFER_HIP_OK) rc = check_linear(L.o_proj, w8, false, hidden, hidden, l, "o_proj");
    if (rc == INFER_HIP_OK) {
      rc = check_linear(L.gate_proj, w8, false, inter, hidden, l, "gate_proj");
    }
    if (rc == INFER_HIP_OK) rc = check_linear(L.up_proj, w8, false, inter, hidden, l, "up_proj");
    if (rc == INFER_HIP_OK) {
      rc = check_linear(L.down_proj, w8, false, hidden, inter, l, "down_proj");
    }
    if (rc != INFER_HIP_OK) return rc;
  }

  auto* m = new (std::nothrow) infer_hip_model();
  if (!m) return fail(INFER_HIP_RUNTIME_ERROR, "model: out of host memory");
  m->cfg = c;
  m->w8 = w8;
  m->use_graph = options->use_graph != 0;
  m->max_seq = max_seq;
  m->head_dim = head_dim;
  m->kv_dim = kv_dim;
  m->embed = weights->embed_tokens;
  m->final_norm = weights->norm;
  m->lm_head = lm_head;
  m->fused_norm_gemv = norm_gemv_supported(hidden, w8);
  m->fused_lm_head = lm_head_decode_supported(hidden);
  m->fused_qkv_rope = m->fused_norm_gemv && attention_whole(max_seq, head_dim) &&
                      norm_qkv_rope_supported(hidden, head_dim, w8) &&
                      attn_o_parts_supported(hidden, w8);
  // The unfused step runs the split attention, which needs head_dim 128 or
  // more than kAttnWholeMax positions; head_dim 64 means at most 32 x 64 =
  // 2048 hidden, always within the fused launches' limits.
  if (attention_whole(max_seq, head_dim) && !m->fused_qkv_rope) {
    destroy_model(m);
    return fail(INFER_HIP_RUNTIME_ERROR, "model: no decode attention form for this shape");
  }

  // Arena layout.
  size_t cursor = 0;
  auto take = [&](size_t bytes) {
    const size_t at = cursor;
    cursor = align_up(cursor + bytes);
    return at;
  };
  const size_t lm_entries = infer_hip_lm_head_workspace_entries(c.vocab_size, hidden);
  const size_t ms = static_cast<size_t>(max_seq);
  const size_t o_state = take(sizeof(ModelState));
  const size_t o_history = take(sizeof(int) * ms);
  const size_t o_prompt = take(sizeof(int) * ms);
  const size_t o_x = take(2 * hidden), o_norm = take(2 * hidden), o_q = take(2 * hidden);
  const size_t o_k = take(2 * kv_dim), o_v = take(2 * kv_dim);
  const size_t o_gate = take(2 * inter), o_up = take(2 * inter), o_mlp = take(2 * inter);
  const size_t o_logits = take(2 * static_cast<size_t>(c.vocab_size));
  const size_t o_lmv = take(sizeof(float) * lm_entries), o_lmi = take(sizeof(int) * lm_entries);
  const size_t o_lmbest = take(8 * static_cast<size_t>(lm_head_decode_blocks(c.vocab_size)));
  const size_t o_lmcounter = take(sizeof(int));
  const size_t o_lmkey = take(sizeof(unsigned long long));
  const size_t o_rope = take(sizeof(float2) * ms * (head_dim / 2));
  const size_t o_rope_cur = take(sizeof(float2) * (head_dim / 2));
  // (the fused step's parts: kDecodeAttnParts records of kAttnPartRecord
  // floats per head)
  const size_t o_partial = take(sizeof(float) * c.num_heads *
                                std::max<size_t>(kDecodeAttnParts * kAttnPartRecord,
                                                 static_cast<size_t>(attention_splits(
                                                     max_seq, head_dim)) * (head_dim + 2)));
  const size_t o_attn = take(2 * hidden);
  const size_t o_px = take(2 * ms * hidden), o_pnorm = take(2 * ms * hidden);
  const size_t o_pq = take(2 * ms * hidden), o_pk = take(2 * ms * kv_dim);
  const size_t o_pv = take(2 * ms * kv_dim), o_pattn = take(2 * ms * hidden);
  const size_t o_ptmp = take(2 * ms * hidden), o_pgate = take(2 * ms * inter);
  const size_t o_pup = take(2 * ms * inter), o_pmlp = take(2 * ms * inter);
  int cus = 0;
  {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) {
      delete m;
      return fail(INFER_HIP_RUNTIME_ERROR, "model: cannot query the device");
    }
  }
  size_t gemm_pf = 0, gemm_cc = 0;
  prefill_scratch_needs(c, head_dim, max_seq, cus, &gemm_pf, &gemm_cc);
  const size_t o_gemm_partial = take(sizeof(float) * gemm_pf);
  const size_t o_gemm_counters = take(sizeof(int) * gemm_cc);
  const size_t o_tables = take(sizeof(W8GroupDesc) * 5 * c.num_layers);
  // One layer's K and V caches, in BF16 elements: [k|v][kv_head][max_seq][head_dim].
  const size_t kv_layer = 2 * static_cast<size_t>(c.num_kv_heads) * ms * head_dim;
  const size_t o_kv = take(2 * kv_layer * c.num_layers);  // bytes
  m->arena_bytes = cursor;
  m->kv_bytes = 2 * kv_layer * c.num_layers;

  hipError_t st = hipGetDevice(&m->device);
  if (st == hipSuccess) st = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking);
  if (st == hipSuccess) st = hipMalloc(reinterpret_cast<void**>(&m->arena), m->arena_bytes);
  if (st == hipSuccess) st = hipMemset(m->arena, 0, m->arena_bytes);
  if (st == hipSuccess) st = hipHostMalloc(reinterpret_cast<void**>(&m->pinned), sizeof(int));
  if (st != hipSuccess) {
    const int rc = hip_fail(st, "model allocation");
    destroy_model(m);
    return rc;
  }
  char* a = m->arena;
  m->state = reinterpret_cast<ModelState*>(a + o_state);
  m->history = reinterpret_cast<int*>(a + o_history);
  m->prompt = reinterpret_cast<int*>(a + o_prompt);
  auto bf = [&](size_t o) { return reinterpret_cast<uint16_t*>(a + o); };
  m->x = bf(o_x); m->norm = bf(o_norm); m->q = bf(o_q); m->k = bf(o_k); m->v = bf(o_v);
  m->gate = bf(o_gate); m->up = bf(o_up); m->mlp = bf(o_mlp);
  m->logits = bf(o_logits);
  m->lm_value = reinterpret_cast<float*>(a + o_lmv);
  m->lm_index = reinterpret_cast<int*>(a + o_lmi);
  m->lm_best = reinterpret_cast<float*>(a + o_lmbest);
  m->lm_counter = reinterpret_cast<int*>(a + o_lmcounter);
  m->lm_key = reinterpret_cast<unsigned long long*>(a + o_lmkey);
  m->rope = reinterpret_cast<float2*>(a + o_rope);
  m->rope_cur = reinterpret_cast<float2*>(a + o_rope_cur);
  m->attn_partial = reinterpret_cast<float*>(a + o_partial);
  m->attn = reinterpret_cast<uint16_t*>(a + o_attn);
  m->px = bf(o_px); m->pnorm = bf(o_pnorm); m->pq = bf(o_pq); m->pk = bf(o_pk); m->pv = bf(o_pv);
  m->pattn = bf(o_pattn); m->ptmp = bf(o_ptmp); m->pgate = bf(o_pgate); m->pup = bf(o_pup);
  m->pmlp = bf(o_pmlp);
  m->cus = cus;
  m->gemm_partial = reinterpret_cast<float*>(a + o_gemm_partial);
  m->gemm_counters = reinterpret_cast<int*>(a + o_gemm_counters);
  m->gemm_partial_floats = gemm_pf;
  m->gemm_counter_count = gemm_cc;
  W8GroupDesc* tables = reinterpret_cast<W8GroupDesc*>(a + o_tables);
  uint16_t* kv = bf(o_kv);

  // RoPE table: (cos, sin) of position * theta^(-2 i / head_dim) in FP32,
  // the CPU path's arithmetic (src/cpu_ops.cpp:38-41).
  const int half = head_dim / 2;
  std::vector<float2> rope(ms * half);
  for (int p = 0; p < max_seq; ++p) {
    for (int i = 0; i < half; ++i) {
      rope[static_cast<size_t>(p) * half + i] = rope_angle(c.rope_theta, head_dim, p, i);
    }
  }
  st = hipMemcpy(m->rope, rope.data(), sizeof(float2) * rope.size(), hipMemcpyHostToDevice);

  // Resolve every layer once; build the grouped-GEMV tables.
  std::vector<W8GroupDesc> host_tables;
  m->layers.resize(c.num_layers);
  for (int l = 0; l < c.num_layers && st == hipSuccess; ++l) {
    const infer_hip_layer_weights& W = weights->layers[l];
    Layer& L = m->layers[l];
    L.in_norm = W.input_layernorm;
    L.post_norm = W.post_attention_layernorm;
    auto lin = [](const infer_hip_linear& w, int n, int k) {
      return Linear{w.weight, w.scales, w.bias, n, k};
    };
    L.q = lin(W.q_proj, hidden, hidden);
    L.k = lin(W.k_proj, kv_dim, hidden);
    L.v = lin(W.v_proj, kv_dim, hidden);
    L.o = lin(W.o_proj, hidden, hidden);
    L.gate = lin(W.gate_proj, inter, hidden);
    L.up = lin(W.up_proj, inter, hidden);
    L.down = lin(W.down_proj, hidden, inter);
    L.key_cache = kv + kv_layer * l;
    L.value_cache = L.key_cache + kv_layer / 2;
    if (w8) {
      auto desc = [&](const Linear& li, const uint16_t* x, uint16_t* y, int& blocks) {
        W8GroupDesc d{static_cast<const int8_t*>(li.w), li.s, li.b, x, y, li.n, li.k, blocks,
                      kDecodeRowsPerBlock};
        blocks += (li.n + kDecodeRowsPerBlock - 1) / kDecodeRowsPerBlock;
        return d;
      };
      L.qkv_table = tables + host_tables.size();
      host_tables.push_back(desc(L.q, m->norm, m->q, L.qkv_blocks));
      host_tables.push_back(desc(L.k, m->norm, m->k, L.qkv_blocks));
      host_tables.push_back(desc(L.v, m->norm, m->v, L.qkv_blocks));
      L.gate_up_table = tables + host_tables.size();
      host_tables.push_back(desc(L.gate, m->norm, m->gate, L.gate_up_blocks));
      host_tables.push_back(desc(L.up, m->norm, m->up, L.gate_up_blocks));
    }
    if (m->fused_norm_gemv) {
      const int gate_up_rows = w8 ? kGateUpRowsPerWave : kGateUpRowsPerWaveBf16;
      auto fdesc = [](const Linear& li, const Linear* pair, uint16_t* y, int rows_per_wave,
                      int& blocks) {
        NormGemvDesc d{li.w, li.s, pair ? pair->w : nullptr, pair ? pair->s : nullptr, li.b, y,
                       li.n, blocks};
        blocks += norm_gemv_blocks(li.n, rows_per_wave);
        return d;
      };
      L.qkv_args = NormGemvArgs{m->x, L.in_norm, c.rms_norm_eps, hidden, 3, kQkvRowsPerWave, {}};
      L.qkv_args.d[0] = fdesc(L.q, nullptr, m->q, kQkvRowsPerWave, L.qkv_fused_blocks);
      L.qkv_args.d[1] = fdesc(L.k, nullptr, m->k, kQkvRowsPerWave, L.qkv_fused_blocks);
      L.qkv_args.d[2] = fdesc(L.v, nullptr, m->v, kQkvRowsPerWave, L.qkv_fused_blocks);
      L.qkv_rope_args = QkvRopeArgs{m->x, L.in_norm, c.rms_norm_eps, hidden,
                                    L.q.w, L.q.s, L.q.b, L.k.w, L.k.s, L.k.b, L.v.w, L.v.s, L.v.b,
                                    m->q, L.key_cache, L.value_cache, m->rope_cur,
                                    &m->state->pos,
                                    c.num_heads, c.num_kv_heads, head_dim, max_seq};
      L.gate_up_args =
          NormGemvArgs{m->x, L.post_norm, c.rms_norm_eps, hidden, 1, gate_up_rows, {}};
      L.gate_up_args.d[0] =
          fdesc(L.gate, &L.up, m->mlp, gate_up_rows, L.gate_up_fused_blocks);
    }
  }
  // Every region the kernels write must lie inside the arena.
  const char* arena_end = m->arena + m->arena_bytes;
  const bool inside =
      reinterpret_cast<const char*>(m->layers.back().value_cache + kv_layer / 2) <= arena_end &&
      reinterpret_cast<const char*>(tables + host_tables.size()) <= a + o_kv &&
      reinterpret_cast<const char*>(m->pmlp + ms * inter) <= a + o_tables;
  if (st == hipSuccess && !inside) {
    destroy_model(m);
    return fail(INFER_HIP_RUNTIME_ERROR, "model: internal arena layout overflow");
  }
  if (st == hipSuccess && !host_tables.empty()) {
    st = hipMemcpy(tables, host_tables.data(), sizeof(W8GroupDesc) * host_tables.size(),
                   hipMemcpyHostToDevice);
  }
  if (st != hipSuccess) {
    const int rc = hip_fail(st, "model set-up");
    destroy_model(m);
    return rc;
  }
  if (m->use_graph) {
    const int rc = ensure_graph(m);
    if (rc != INFER_HIP_OK) {
      destroy_model(m);
      return rc;
    }
  }
  *out = m;
  return ok();
}

extern "C" int infer_hip_model_destroy(infer_hip_model* model) {
  destroy_model(model);
  return ok();
}

namespace {

// Closes the archive on every exit of infer_hip_model_open.
struct ArchiveHandle {
  infer_hip_archive* a = nullptr;
  ~ArchiveHandle() { (void)infer_hip_archive_close(a); }
};

// Record `name` with the given dtype and shape, or an error naming it.
int expect_record(const infer_hip_archive* a, const std::string& name, int dtype,
                  std::initializer_list<int64_t> shape, infer_hip_tensor_record* rec) {
  const int i = infer_hip_archive_find(a, name.c_str());
  if (i < 0) return fail(INFER_HIP_INVALID_ARGUMENT, "missing tensor: %s", name.c_str());
  int rc = infer_hip_archive_record(a, i, rec);
  if (rc != INFER_HIP_OK) return rc;
  bool same = rec->dtype == dtype && rec->ndim == static_cast<int>(shape.size());
  int d = 0;
  for (int64_t v : shape) same = same && rec->shape[d++] == v;
  if (!same) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "tensor %s: unexpected dtype or shape",
                name.c_str());
  }
  return ok();
}

}  // namespace

// Qwen2Model::Qwen2Model(model_directory, options) and initialize_weights
// (src/qwen2.cpp:30-78): every record goes into one device allocation, each
// at a 256-byte aligned offset in file order; the Linear tensors are then
// resolved by their archive names (src/qwen2.cpp:606-660) and the scale
// tensor of a quantised weight through its "quant" record.
extern "C" int infer_hip_model_open(const char* model_directory,
                                    const infer_hip_runtime_options* options,
                                    infer_hip_model** out) {
  if (!out) return fail(INFER_HIP_INVALID_ARGUMENT, "model: null output pointer");
  *out = nullptr;
  if (!model_directory || !options) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "model: null directory or options");
  }
  const std::string dir = model_directory;
  infer_hip_model_config cfg{};
  int max_positions = 0;
  int rc = infer_hip_model_config_load((dir + "/config.json").c_str(), &cfg, &max_positions);
  if (rc != INFER_HIP_OK) return rc;
  if (options->max_sequence_length <= 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "max sequence length must be positive");
  }
  if (options->max_sequence_length > max_positions) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "max sequence length exceeds model limit");
  }
  const bool w8 = options->precision == INFER_HIP_PRECISION_W8A16;
  if (!w8 && options->precision != INFER_HIP_PRECISION_W16A16) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "model: precision must be W16A16 or W8A16 (the FP32 path is the CPU's)");
  }
  // archive_filename (include/infer/common.hpp:49-55)
  const std::string file = dir + (w8 ? "/model.w8a16.qbin" : "/model.w16a16.qbin");
  ArchiveHandle archive;
  rc = infer_hip_archive_open(file.c_str(), &archive.a);
  if (rc != INFER_HIP_OK) return rc;
  const infer_hip_archive* a = archive.a;

  // Device layout: one allocation, each record at a 256-byte aligned offset.
  const int count = infer_hip_archive_tensor_count(a);
  std::vector<size_t> offsets(count);
  size_t total = 0;
  for (int i = 0; i < count; ++i) {
    infer_hip_tensor_record r;
    rc = infer_hip_archive_record(a, i, &r);
    if (rc != INFER_HIP_OK) return rc;
    total = align_up(total);
    offsets[i] = total;
    total += r.nbytes;
  }

  const int hidden = cfg.hidden_size, inter = cfg.intermediate_size;
  const int head_dim = hidden / cfg.num_heads;  // the config loader checked divisibility
  const int kv_dim = cfg.num_kv_heads * head_dim;
  infer_hip_model_weights weights{};
  std::vector<infer_hip_layer_weights> layers(cfg.num_layers);
  // Resolves every weight the model needs against `base`; run once with
  // base 0 to validate names, dtypes and shapes before any allocation, then
  // with the device allocation.
  auto resolve = [&](uintptr_t base) {
    infer_hip_tensor_record r;
    auto at = [&](const infer_hip_tensor_record& rec) {
      return reinterpret_cast<const void*>(base + offsets[infer_hip_archive_find(a, rec.name)]);
    };
    auto bf16_vector = [&](const std::string& name, int64_t n, const uint16_t** p) {
      const int e = expect_record(a, name, INFER_HIP_DTYPE_BFLOAT16, {n}, &r);
      if (e == INFER_HIP_OK) *p = static_cast<const uint16_t*>(at(r));
      return e;
    };
    auto linear = [&](const std::string& name, int64_t n, int64_t k, bool bias,
                      infer_hip_linear* l) {
      *l = infer_hip_linear{};
      int e = expect_record(a, name + ".weight",
                            w8 ? INFER_HIP_DTYPE_INT8 : INFER_HIP_DTYPE_BFLOAT16, {n, k}, &r);
      if (e != INFER_HIP_OK) return e;
      l->weight = at(r);
      if (w8) {
        if (r.quant_group_size != 64 || r.quant_axis != 1 || !r.scale_tensor) {
          return fail(INFER_HIP_INVALID_ARGUMENT,
                      "tensor %s.weight: expected group-64 quantisation", name.c_str());
        }
        const std::string scale = r.scale_tensor;
        e = expect_record(a, scale, INFER_HIP_DTYPE_BFLOAT16, {n, (k + 63) / 64}, &r);
        if (e != INFER_HIP_OK) return e;
        l->scales = static_cast<const uint16_t*>(at(r));
      }
      return bias ? bf16_vector(name + ".bias", n, &l->bias) : ok();
    };
    weights = infer_hip_model_weights{};
    int e = expect_record(a, "model.embed_tokens.weight", INFER_HIP_DTYPE_BFLOAT16,
                          {cfg.vocab_size, hidden}, &r);
    if (e != INFER_HIP_OK) return e;
    weights.embed_tokens = static_cast<const uint16_t*>(at(r));
    e = bf16_vector("model.norm.weight", hidden, &weights.norm);
    if (e == INFER_HIP_OK && infer_hip_archive_find(a, "lm_head.weight") >= 0) {
      e = expect_record(a, "lm_head.weight", INFER_HIP_DTYPE_BFLOAT16, {cfg.vocab_size, hidden},
                        &r);
      if (e == INFER_HIP_OK) weights.lm_head = static_cast<const uint16_t*>(at(r));
    }
    for (int l = 0; l < cfg.num_layers && e == INFER_HIP_OK; ++l) {
      const std::string p = "model.layers." + std::to_string(l) + ".";
      infer_hip_layer_weights& L = layers[l];
      e = bf16_vector(p + "input_layernorm.weight", hidden, &L.input_layernorm);
      if (e == INFER_HIP_OK) {
        e = bf16_vector(p + "post_attention_layernorm.weight", hidden,
                        &L.post_attention_layernorm);
      }
      if (e == INFER_HIP_OK) e = linear(p + "self_attn.q_proj", hidden, hidden, true, &L.q_proj);
      if (e == INFER_HIP_OK) e = linear(p + "self_attn.k_proj", kv_dim, hidden, true, &L.k_proj);
      if (e == INFER_HIP_OK) e = linear(p + "self_attn.v_proj", kv_dim, hidden, true, &L.v_proj);
      if (e == INFER_HIP_OK) e = linear(p + "self_attn.o_proj", hidden, hidden, false, &L.o_proj);
      if (e == INFER_HIP_OK) e = linear(p + "mlp.gate_proj", inter, hidden, false, &L.gate_proj);
      if (e == INFER_HIP_OK) e = linear(p + "mlp.up_proj", inter, hidden, false, &L.up_proj);
      if (e == INFER_HIP_OK) e = linear(p + "mlp.down_proj", hidden, inter, false, &L.down_proj);
    }
    weights.layers = layers.data();
    return e;
  };
  rc = resolve(0);
  if (rc != INFER_HIP_OK) return rc;

  char* device = nullptr;
  hipError_t st = hipMalloc(reinterpret_cast<void**>(&device), std::max<size_t>(total, 256));
  if (st != hipSuccess) return hip_fail(st, "model weight allocation");
  for (int i = 0; i < count && st == hipSuccess; ++i) {
    infer_hip_tensor_record r;
    (void)infer_hip_archive_record(a, i, &r);
    if (r.nbytes) {
      st = hipMemcpy(device + offsets[i], infer_hip_archive_data(a, i), r.nbytes,
                     hipMemcpyHostToDevice);
    }
  }
  if (st != hipSuccess) {
    (void)hipFree(device);
    return hip_fail(st, "model weight upload");
  }
  rc = resolve(reinterpret_cast<uintptr_t>(device));
  infer_hip_model* m = nullptr;
  if (rc == INFER_HIP_OK) rc = infer_hip_model_create(&cfg, &weights, options, &m);
  if (rc != INFER_HIP_OK) {
    (void)hipFree(device);
    return rc;
  }
  m->owned_weights = device;
  *out = m;
  return ok();
}

extern "C" int infer_hip_model_reset(infer_hip_model* m) {
  if (!m) return fail(INFER_HIP_INVALID_ARGUMENT, "model: null model");
  m->position = 0;
  m->has_prefilled = false;
  m->last_token = -1;
  return ok();
}

extern "C" int infer_hip_model_prefill(infer_hip_model* m, const int* tokens, int count,
                                       int* next_token) {
  if (!m || !next_token) return fail(INFER_HIP_INVALID_ARGUMENT, "prefill: null argument");
  if (!tokens || count <= 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "prompt must contain at least one token");
  }
  if (m->position != 0 || m->has_prefilled) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "prefill requires a fresh model state; call reset first");
  }
  if (count > m->max_seq) return fail(INFER_HIP_INVALID_ARGUMENT, "prompt exceeds KV cache capacity");
  for (int i = 0; i < count; ++i) {
    if (tokens[i] < 0 || tokens[i] >= m->cfg.vocab_size) {
      return fail(INFER_HIP_INVALID_ARGUMENT, "input token out of range");
    }
  }
  DeviceGuard guard(m->device);
  const int rc = run_prefill(m, tokens, count, next_token);
  if (rc != INFER_HIP_OK) return rc;
  m->position = count;
  m->has_prefilled = true;
  m->last_token = *next_token;
  return ok();
}

extern "C" int infer_hip_model_decode_next(infer_hip_model* m, int token, int* next_token) {
  if (!m || !next_token) return fail(INFER_HIP_INVALID_ARGUMENT, "decode_next: null argument");
  if (!m->has_prefilled) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "decode_next requires a successful prefill");
  }
  if (token < 0 || token >= m->cfg.vocab_size) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "input token out of range");
  }
  if (m->position >= m->max_seq) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "KV cache capacity exceeded");
  }
  DeviceGuard guard(m->device);
  launch_set_state(m->state, token, m->position, 0, rope_cursor(m), m->stream, m->lm_key);
  int rc = check_launch("decode state");
  if (rc == INFER_HIP_OK) rc = run_decode_step(m);
  if (rc == INFER_HIP_OK) rc = finish_decode(m);
  if (rc == INFER_HIP_OK) rc = read_token(m, next_token);
  if (rc != INFER_HIP_OK) return rc;
  ++m->position;
  m->last_token = *next_token;
  return ok();
}

extern "C" int infer_hip_model_rewind(infer_hip_model* m, int position, int token) {
  if (!m) return fail(INFER_HIP_INVALID_ARGUMENT, "rewind: null model");
  if (!m->has_prefilled) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "rewind requires a successful prefill");
  }
  if (position < 1 || position > m->position) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "rewind: position %d outside [1, %d]", position,
                m->position);
  }
  if (token < 0 || token >= m->cfg.vocab_size) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "input token out of range");
  }
  // Every decode entry point sets the device state from these two values
  // before its first step, so nothing on the device needs to change here.
  m->position = position;
  m->last_token = token;
  return ok();
}

extern "C" int infer_hip_model_decode_steps(infer_hip_model* m, int steps, int* tokens_out) {
  if (!m) return fail(INFER_HIP_INVALID_ARGUMENT, "decode_steps: null model");
  if (!m->has_prefilled) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "decode_steps requires a successful prefill");
  }
  if (steps < 0 || m->position + static_cast<long long>(steps) > m->max_seq) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "KV cache capacity exceeded");
  }
  if (steps == 0) return ok();
  DeviceGuard guard(m->device);
  launch_set_state(m->state, m->last_token, m->position, 0, rope_cursor(m), m->stream,
                   m->lm_key);
  int rc = check_launch("decode state");
  for (int i = 0; i < steps && rc == INFER_HIP_OK; ++i) rc = run_decode_step(m);
  if (rc == INFER_HIP_OK) rc = finish_decode(m);
  if (rc != INFER_HIP_OK) return rc;
  hipError_t st = hipSuccess;
  if (tokens_out) {
    st = hipMemcpyAsync(tokens_out, m->history, sizeof(int) * steps, hipMemcpyDeviceToHost,
                        m->stream);
  }
  if (st != hipSuccess) return hip_fail(st, "decode history readback");
  int last = 0;
  rc = read_token(m, &last);  // synchronizes
  if (rc != INFER_HIP_OK) return rc;
  m->position += steps;
  m->last_token = last;
  return ok();
}

extern "C" int infer_hip_model_generate(infer_hip_model* m, const int* prompt, int prompt_count,
                                        int max_new_tokens, int stop_on_eos, int* tokens_out,
                                        int* generated, infer_hip_generation_stats* stats) {
  if (!m || !prompt || !generated || (max_new_tokens > 0 && !tokens_out)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "generate: null argument");
  }
  if (prompt_count <= 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "prompt must contain at least one token");
  }
  if (max_new_tokens < 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "max_new_tokens must be non-negative");
  }
  if (static_cast<long long>(prompt_count) + std::max(0, max_new_tokens - 1) > m->max_seq) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "prompt and generation exceed KV cache capacity");
  }
  *generated = 0;
  infer_hip_model_reset(m);
  const double t0 = now_ms();
  int next = 0;
  int rc = infer_hip_model_prefill(m, prompt, prompt_count, &next);
  if (rc != INFER_HIP_OK) return rc;
  const double t1 = now_ms();
  int count = 0;
  if (max_new_tokens > 0) tokens_out[count++] = next;
  const int eos = m->cfg.eos_token_id;
  // Without EOS stopping the whole decode is one host-sync-free run; with
  // it, runs of kEosChunk steps are checked between runs (the steps after
  // an EOS inside a run are discarded, and the position is set back).
  constexpr int kEosChunk = 16;
  bool stopped = stop_on_eos && count > 0 && tokens_out[count - 1] == eos;
  while (count < max_new_tokens && !stopped) {
    const int steps = stop_on_eos ? std::min(kEosChunk, max_new_tokens - count)
                                  : max_new_tokens - count;
    const int base_position = m->position;
    rc = infer_hip_model_decode_steps(m, steps, tokens_out + count);
    if (rc != INFER_HIP_OK) return rc;
    if (stop_on_eos) {
      for (int i = 0; i < steps; ++i) {
        if (tokens_out[count + i] == eos) {
          m->position = base_position + i + 1;
          m->last_token = eos;
          count += i + 1;
          stopped = true;
          break;
        }
      }
    }
    if (!stopped) count += steps;
  }
  const double t2 = now_ms();
  *generated = count;
  if (stats) {
    stats->prompt_tokens = prompt_count;
    stats->generated_tokens = count;
    stats->ttft_ms = t1 - t0;
    stats->decode_ms = t2 - t1;
    stats->total_ms = t2 - t0;
  }
  return ok();
}

extern "C" int infer_hip_model_last_logits(infer_hip_model* m, float* logits) {
  if (!m || !logits) return fail(INFER_HIP_INVALID_ARGUMENT, "last_logits: null argument");
  DeviceGuard guard(m->device);
  std::vector<uint16_t> bits(static_cast<size_t>(m->cfg.vocab_size));
  hipError_t st = hipMemcpyAsync(bits.data(), m->logits, sizeof(uint16_t) * bits.size(),
                                 hipMemcpyDeviceToHost, m->stream);
  if (st == hipSuccess) st = hipStreamSynchronize(m->stream);
  if (st != hipSuccess) return hip_fail(st, "logits readback");
  for (size_t i = 0; i < bits.size(); ++i) {
    const uint32_t word = static_cast<uint32_t>(bits[i]) << 16;
    std::memcpy(logits + i, &word, sizeof(float));
  }
  return ok();
}

extern "C" int infer_hip_model_position(const infer_hip_model* m) { return m ? m->position : -1; }

extern "C" int infer_hip_model_has_prefilled(const infer_hip_model* m) {
  return m && m->has_prefilled ? 1 : 0;
}

extern "C" size_t infer_hip_model_kv_cache_bytes(const infer_hip_model* m) {
  return m ? m->kv_bytes : 0;
}

extern "C" size_t infer_hip_model_workspace_bytes(const infer_hip_model* m) {
  return m ? m->arena_bytes - m->kv_bytes : 0;
}

extern "C" hipStream_t infer_hip_model_stream(const infer_hip_model* m) {
  return m ? m->stream : nullptr;
}

extern "C" int infer_hip_attention_prefill_bf16(const uint16_t* q, const uint16_t* key_cache,
                                                const uint16_t* value_cache, uint16_t* output,
                                                int token_count, int num_heads, int num_kv_heads,
                                                int head_dim, int max_sequence_length,
                                                hipStream_t stream) {
  if (!q || !key_cache || !value_cache || !output) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "attention_prefill: null pointer");
  }
  if (token_count <= 0 || token_count > max_sequence_length || num_heads <= 0 ||
      num_kv_heads <= 0 || num_heads % num_kv_heads != 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "attention_prefill: bad shape (tokens %d, heads %d / %d, max_seq %d)",
                token_count, num_heads, num_kv_heads, max_sequence_length);
  }
  if (!attention_head_dim_supported(head_dim)) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "attention_prefill: head_dim %d unsupported (64 or 128)",
                head_dim);
  }
  launch_attention_prefill(q, key_cache, value_cache, output, token_count, num_heads,
                           num_kv_heads, head_dim, max_sequence_length, stream);
  return check_launch("attention_prefill");
}

extern "C" const char* infer_hip_model_kernel_name(int kind) {
  return kind >= 0 && kind < kKindCount ? kKindNames[kind] : nullptr;
}

extern "C" int infer_hip_model_kernel_times(infer_hip_model* m, int position, int reps,
                                            double* us, double* bytes, int* launches,
                                            int count) {
  if (!m || !us || !bytes || !launches || count < kKindCount || reps <= 0) {
    return fail(INFER_HIP_INVALID_ARGUMENT, "kernel_times: bad argument");
  }
  if (!m->has_prefilled || position < 1 || position >= m->max_seq || position > m->position) {
    return fail(INFER_HIP_INVALID_ARGUMENT,
                "kernel_times: position must lie in [1, current position] of a prefilled model");
  }
  DeviceGuard guard(m->device);
  hipEvent_t start = nullptr, stop = nullptr;
  hipError_t st = hipEventCreate(&start);
  if (st == hipSuccess) st = hipEventCreate(&stop);
  int rc = st == hipSuccess ? ok() : hip_fail(st, "kernel_times events");
  for (int kind = 0; kind < kKindCount && rc == INFER_HIP_OK; ++kind) {
    bytes[kind] = kind_bytes(m, kind, position + 1, &launches[kind]);
    us[kind] = 0.0;
    if (launches[kind] == 0) continue;
    bytes[kind] /= launches[kind];
    // The kind's launches of one step, captured as a graph (as the decode
    // step runs them) and replayed `reps` times between two events.  Kinds
    // with few launches per step (embedding, LM head) are captured several
    // times over, so that the graph launch's own overhead is shared by some
    // 24 kernels as in the decode step, not charged to one.
    const int copies = std::max(1, (24 + launches[kind] - 1) / launches[kind]);
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    st = hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal);
    if (st != hipSuccess) {
      rc = hip_fail(st, "kernel_times capture");
      break;
    }
    for (int c = 0; c < copies && rc == INFER_HIP_OK; ++c) rc = enqueue_decode_step(m, kind);
    st = hipStreamEndCapture(m->stream, &graph);
    if (rc == INFER_HIP_OK && st != hipSuccess) rc = hip_fail(st, "kernel_times capture");
    if (rc == INFER_HIP_OK) {
      st = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
      if (st != hipSuccess) rc = hip_fail(st, "kernel_times instantiate");
    }
    if (rc == INFER_HIP_OK) {
      launch_set_state(m->state, m->last_token, position, 0, rope_cursor(m), m->stream,
                       m->lm_key);
      st = hipGraphLaunch(exec, m->stream);  // warm-up
      if (st == hipSuccess) st = hipEventRecord(start, m->stream);
      for (int r = 0; r < reps && st == hipSuccess; ++r) st = hipGraphLaunch(exec, m->stream);
      if (st == hipSuccess) st = hipEventRecord(stop, m->stream);
      if (st == hipSuccess) st = hipEventSynchronize(stop);
      float ms = 0.0f;
      if (st == hipSuccess) st = hipEventElapsedTime(&ms, start, stop);
      if (st != hipSuccess) {
        rc = hip_fail(st, "kernel_times");
      } else {
        us[kind] = ms * 1e3 / (static_cast<double>(reps) * copies * launches[kind]);
      }
    }
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
  }
  if (start) (void)hipEventDestroy(start);
  if (stop) (void)hipEventDestroy(stop);
  // The replays rewrote the KV-cache row at `position` and the activations:
  // the model needs a fresh prefill.
  m->position = 0;
  m->has_prefilled = false;
  return rc;
}
