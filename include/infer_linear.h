/*
 * C ABI of the MI355X (gfx950) Linear hot path: W8A16 group-64 dequant
 * GEMV/GEMM, BF16 W16A16 GEMV/GEMM, and the fused tied-embedding LM head
 * with argmax.
 *
 * Each entry point replaces one free function of the reference's operator
 * boundary, include/infer/cuda_ops.hpp (Greedy-cy/qwen2.5-jetson-inference),
 * with the same argument order and meaning:
 *   - pointers are caller-owned device memory (no allocation inside an op);
 *   - BF16 tensors are passed as their 16-bit words (uint16_t);
 *   - weights are row-major [out_features, in_features]; W8A16 scales are
 *     BF16 [out_features, ceil(in_features / 64)], group g covering columns
 *     [64 g, 64 g + 64) (tools/export_model.py:228-242);
 *   - activations are [tokens, in_features], outputs [tokens, out_features],
 *     FP32 accumulation, BF16 round-to-nearest-even output;
 *   - bias may be NULL;
 *   - work is enqueued on `stream` and never synchronised (the caller syncs
 *     before reading results, as src/qwen2.cpp:668-673 does).
 * Where the reference throws infer::Error (INFER_CHECK / INFER_CUDA_CHECK,
 * include/infer/common.hpp:66-82) these return a nonzero status and leave a
 * message for infer_hip_last_error(); they never throw.
 *
 * Fast paths need 16-byte aligned weight and activation pointers and
 * in_features % 64 == 0 (W8A16) or % 8 == 0 (BF16); anything else runs an
 * exact-semantics fallback kernel, as the reference's scalar kernels do.
 */
#ifndef INFER_LINEAR_H
#define INFER_LINEAR_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define INFER_HIP_ABI_VERSION 1

enum infer_hip_status {
  INFER_HIP_OK = 0,
  INFER_HIP_INVALID_ARGUMENT = 1, /* reference: INFER_CHECK throws */
  INFER_HIP_LAUNCH_FAILED = 2,    /* reference: INFER_CUDA_CHECK throws */
  INFER_HIP_RUNTIME_ERROR = 3     /* a HIP runtime call other than a launch */
};

/* Message for the last nonzero status returned on this thread ("" if the
 * last call succeeded). */
const char* infer_hip_last_error(void);

/* INFER_HIP_ABI_VERSION of the loaded library. */
int infer_hip_abi_version(void);

/* y[n] = bf16(sum_k W[n,k] x[k] + bias[n]).
 * Replaces infer::cuda::gemv_bf16, include/infer/cuda_ops.hpp:24-26
 * (launcher src/cuda/kernels.cu:1540-1564). */
int infer_hip_gemv_bf16(const uint16_t* weight, const uint16_t* bias,
                        const uint16_t* input, uint16_t* output,
                        int out_features, int in_features, hipStream_t stream);

/* Y[m,n] = bf16(sum_k X[m,k] W[n,k] + bias[n]) for m < tokens.
 * Replaces infer::cuda::gemm_bf16, include/infer/cuda_ops.hpp:32-35
 * (launcher src/cuda/kernels.cu:1600-1625). */
int infer_hip_gemm_bf16(const uint16_t* weight, const uint16_t* bias,
                        const uint16_t* input, uint16_t* output, int tokens,
                        int out_features, int in_features, hipStream_t stream);

/* Tied LM head: logits[v] = bf16(E[v,:] h + bias[v]) for v < vocab, and
 * *argmax = the first index of the maximum of the FP32 sums (ties -> lowest
 * index, the CPU path's std::max_element, src/cpu_ops.cpp:175-177).
 * block_max_value / block_max_index are scratch of at least
 * infer_hip_lm_head_workspace_entries(vocab, in_features) entries each; that
 * count never exceeds ceil(vocab / 8), the reference's sizing
 * (src/qwen2.cpp:193-198).
 * Replaces infer::cuda::lm_head_bf16, include/infer/cuda_ops.hpp:42-45
 * (launcher src/cuda/kernels.cu:1566-1579).  Difference: the reference
 * takes the argmax over BF16-rounded logits (kernels.cu:545-547); this one
 * takes it over the FP32 sums so that it equals the CPU FP32 argmax. */
int infer_hip_lm_head_bf16(const uint16_t* weight, const uint16_t* bias,
                           const uint16_t* input, uint16_t* logits,
                           float* block_max_value, int* block_max_index,
                           int* argmax, int vocab, int in_features,
                           hipStream_t stream);

/* infer_hip_lm_head_bf16 without the workspace arguments: the first-stage
 * block winners go to a static device array of the library (65536 (value,
 * index) pairs, 512 KiB per GPU, held until the process ends) instead of
 * caller memory, so the call allocates nothing and needs nothing but its
 * inputs and outputs.  No counterpart in the reference: it is for callers
 * that cannot allocate or size a workspace (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Limit:
 * infer_hip_lm_head_workspace_entries(vocab, in_features) <= 65536, which
 * holds for every vocab <= 1048576; larger shapes return
 * INFER_HIP_INVALID_ARGUMENT.  All calls on one GPU share its array: calls
 * that overlap on one GPU (concurrent streams, threads) race.  Each call
 * writes every entry it reads, so nothing needs clearing between calls.
 * The stream must belong to the current device. */
int infer_hip_lm_head_bf16_noalloc(const uint16_t* weight, const uint16_t* bias,
                                   const uint16_t* input, uint16_t* logits, int* argmax,
                                   int vocab, int in_features, hipStream_t stream);

/* Entries of block_max_value / block_max_index infer_hip_lm_head_bf16 uses
 * for this shape (0 for invalid shapes).  No reference counterpart: the
 * reference sizes its workspace inline (src/qwen2.cpp:193-198). */
size_t infer_hip_lm_head_workspace_entries(int vocab, int in_features);

/* y[n] = bf16(sum_k q[n,k] * s[n, k/64] * x[k] + bias[n]), FP32 sums; the
 * dequantised weight q*s is exact in FP32.  group_size must be 64.
 * Replaces infer::cuda::gemv_w8a16, include/infer/cuda_ops.hpp:47-50
 * (launcher src/cuda/kernels.cu:1627-1655). */
int infer_hip_gemv_w8a16(const int8_t* weight, const uint16_t* scales,
                         int group_size, const uint16_t* bias,
                         const uint16_t* input, uint16_t* output,
                         int out_features, int in_features, hipStream_t stream);

/* Y[m,n] = bf16(sum_k q[n,k] * s[n, k/64] * X[m,k] + bias[n]) for m < tokens.
 * group_size must be 64.  The group scale is applied to the FP32 partial sum
 * of each 64-column group, so the product uses the exact dequantised weight
 * (the reference rounds q*s to BF16 first, kernels.cu:1091).
 * Replaces infer::cuda::gemm_w8a16, include/infer/cuda_ops.hpp:51-55
 * (launcher src/cuda/kernels.cu:1657-1684). */
int infer_hip_gemm_w8a16(const int8_t* weight, const uint16_t* scales,
                         int group_size, const uint16_t* bias,
                         const uint16_t* input, uint16_t* output, int tokens,
                         int out_features, int in_features, hipStream_t stream);

/* ---- Explicit MFMA tile selection --------------------------------------
 * No reference counterpart (the reference picks its WMMA tile from M and N
 * divisibility, src/cuda/kernels.cu:1606-1622, 1665-1681).  The same
 * computation as infer_hip_gemm_w8a16 / infer_hip_gemm_bf16 with the
 * workgroup tile of the MFMA kernel named by the caller: tile in
 * [0, infer_hip_gemm_tile_count()) (0 = 128x128, 1 = 128x64, 2 = 64x128,
 * 3 = 64x64, 4 = 32x128, 5 = 256x128 with 8 waves, rows x columns of Y),
 * or -1 for the automatic choice the plain entry points make (which for a
 * few tokens — 2 to 32, more for narrow or int8 shapes — is the skinny
 * kernel: 32 weight rows per workgroup streamed once, no tile).  For
 * tuning sweeps and for tests that cover every tile.  Shapes outside the
 * MFMA path (tokens == 1, in_features % 64 != 0, unaligned weight or input)
 * ignore tile. */
int infer_hip_gemm_tile_count(void);
int infer_hip_gemm_w8a16_tile(const int8_t* weight, const uint16_t* scales,
                              int group_size, const uint16_t* bias,
                              const uint16_t* input, uint16_t* output, int tokens,
                              int out_features, int in_features, int tile,
                              hipStream_t stream);
int infer_hip_gemm_bf16_tile(const uint16_t* weight, const uint16_t* bias,
                             const uint16_t* input, uint16_t* output, int tokens,
                             int out_features, int in_features, int tile,
                             hipStream_t stream);

/* ---- Lone GEMMs with a caller workspace ---------------------------------
 * No reference counterpart: for a caller that keeps the reference's
 * one-call-per-Linear prefill (src/qwen2.cpp:300-330) and can hold a
 * workspace, as Qwen2Model holds its LM-head scratch (qwen2.cpp:191-199).
 * The same computation as infer_hip_gemm_w8a16 / infer_hip_gemm_bf16; a
 * GEMM whose lone launch would leave CUs idle on a long K (down_proj,
 * K = 4864, at tokens <= 512) is split over K in parts whose FP32 partial
 * tiles go to the workspace and are summed in part order (up to 4 parts of
 * 64 x 64 tiles; with few tokens, where the call runs the skinny kernel,
 * parts of at most 16 groups of 64 per 32-row block and 32-token tile).
 *
 * infer_hip_gemm_workspace_bytes: bytes that cover every token count from 2
 * to max_tokens for this [out_features, in_features] weight on the current
 * device (0: no such call splits); a workspace shared by several weights
 * needs the sum of theirs.  The workspace (device memory, 16-byte aligned)
 * must be zeroed once before its first use; every call leaves it ready for
 * the next (its arrival counters sit at fixed places and return to zero).
 * Calls that share a workspace must not overlap (one stream, or ordered
 * across streams).  A workspace smaller than a call needs is rejected
 * (status 1); null with 0 bytes is accepted for calls that do not split. */
size_t infer_hip_gemm_workspace_bytes(int max_tokens, int out_features, int in_features);
int infer_hip_gemm_w8a16_ws(const int8_t* weight, const uint16_t* scales, int group_size,
                            const uint16_t* bias, const uint16_t* input, uint16_t* output,
                            int tokens, int out_features, int in_features, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);
int infer_hip_gemm_bf16_ws(const uint16_t* weight, const uint16_t* bias, const uint16_t* input,
                           uint16_t* output, int tokens, int out_features, int in_features,
                           void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ---- Grouped W8A16 GEMV plans ------------------------------------------
 * No single reference counterpart: a plan is the multi-matrix form of
 * infer_hip_gemv_w8a16 for GEMVs that are independent of each other, such
 * as q/k/v on one normed input and gate/up on another (src/qwen2.cpp:
 * 615-626, 646-651 issue them as separate gemv_w8a16 calls), or a sweep
 * over many layers' Linears (tools/linear_benchmark.cpp measures them one
 * by one).  Each descriptor has the meaning of one infer_hip_gemv_w8a16
 * call and must meet its fast-path preconditions (group_size 64,
 * in_features % 64 == 0 and <= 8192, 16-byte aligned weight and input);
 * no output may alias any input of the same plan.  create resolves and
 * uploads the descriptor table once (it allocates device memory on the
 * current device); launch enqueues one kernel per K class and allocates
 * nothing. */
typedef struct infer_hip_w8a16_gemv_desc {
  const int8_t* weight;
  const uint16_t* scales;
  int group_size;
  const uint16_t* bias;
  const uint16_t* input;
  uint16_t* output;
  int out_features;
  int in_features;
} infer_hip_w8a16_gemv_desc;

typedef struct infer_hip_gemv_plan infer_hip_gemv_plan;

int infer_hip_w8a16_gemv_plan_create(const infer_hip_w8a16_gemv_desc* descs,
                                     int count, infer_hip_gemv_plan** plan);
int infer_hip_w8a16_gemv_plan_launch(const infer_hip_gemv_plan* plan,
                                     hipStream_t stream);
/* Compulsory bytes one launch moves: weights, scales, inputs, outputs and
 * biases of every descriptor. */
double infer_hip_w8a16_gemv_plan_bytes(const infer_hip_gemv_plan* plan);
int infer_hip_w8a16_gemv_plan_destroy(infer_hip_gemv_plan* plan);

/* ---- Grouped GEMM plans (prefill) --------------------------------------
 * No single reference counterpart: the multi-matrix form of
 * infer_hip_gemm_w8a16 / infer_hip_gemm_bf16 for GEMMs independent of
 * each other, such as q/k/v on one normed input and gate/up on another
 * (src/qwen2.cpp:526-571 issues them as separate gemm_w8a16 calls), or a
 * sweep over a layer's Linears (tools/linear_benchmark.cpp measures them
 * one by one).  Each descriptor has the meaning of one
 * infer_hip_gemm_w8a16 (w8a16 = 1: weight is int8 with BF16 group-64
 * scales) or infer_hip_gemm_bf16 (w8a16 = 0: weight is BF16, scales and
 * group_size ignored) call; all descriptors of a plan have the same
 * w8a16 value.  Each must meet the MFMA path's preconditions:
 * tokens >= 2, in_features % 64 == 0, 16-byte aligned weight and input,
 * every operand under 2 GiB; no output may alias any input of the same
 * plan.  create resolves and uploads the descriptor table once (it
 * allocates device memory on the current device: the table and, when some
 * reduction is split, FP32 partial tiles); launch enqueues one kernel and
 * allocates nothing.  A descriptor whose K is much longer than the plan's
 * shortest is split over K into parts of about that length, summed in a
 * fixed order (results do not depend on scheduling); the longest units
 * start first.  Launches of one plan must not overlap (they share the
 * partial tiles): keep them on one stream. */
typedef struct infer_hip_gemm_desc {
  int w8a16;
  const void* weight;
  const uint16_t* scales;
  int group_size;
  const uint16_t* bias;
  const uint16_t* input;
  uint16_t* output;
  int tokens;
  int out_features;
  int in_features;
} infer_hip_gemm_desc;

typedef struct infer_hip_gemm_plan infer_hip_gemm_plan;

int infer_hip_gemm_plan_create(const infer_hip_gemm_desc* descs, int count,
                               infer_hip_gemm_plan** plan);
int infer_hip_gemm_plan_launch(const infer_hip_gemm_plan* plan, hipStream_t stream);
/* 2 * tokens * out_features * in_features summed over the descriptors. */
double infer_hip_gemm_plan_flops(const infer_hip_gemm_plan* plan);
int infer_hip_gemm_plan_destroy(infer_hip_gemm_plan* plan);

/* Measurement hook, no counterpart in the reference: launches a plan on the
 * 256 x 128 tile (every descriptor with 256 tokens or more) with each
 * workgroup of its GEMM launch writing 16 words to stamps[16 w .. 16 w + 15]
 * (device memory): entry, first stage loaded, epilogue start and end, in
 * 100 MHz ticks; the XCC_ID and HW_ID hardware registers; the unit
 * (logical block | stages << 16 | kind << 24, kind 0 whole tile, 1 split
 * part, 2 gate|up pair); the shader-clock cycles from entry to end; for a
 * split part handing off inside the launch, the times its FP32 tile was
 * stored, every part had arrived and its slices were summed (else 0);
 * words 11-15 are 0.
 * *workgroups receives the launch's workgroup count; with stamps null the
 * call only reports it.  Results are the plan's.  Fails with
 * INFER_HIP_INVALID_ARGUMENT on other plans or when capacity (workgroups)
 * is too small. */
int infer_hip_gemm_plan_timeline(const infer_hip_gemm_plan* plan, unsigned long long* stamps,
                                 int capacity, int* workgroups, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* INFER_LINEAR_H */
