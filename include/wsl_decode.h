/*
 * wsl_decode.h — decode-step kernels of the weight-shared Qwen3 harness (libwsl.so).
 *
 * These have no counterpart at the reference's boundary: the reference runs them as torch
 * ops inside its Qwen3 block (torchtitan/experiments/qwen3/model/model.py:167-218,
 * 250-251, 296-314) and re-runs the whole prefix every generated token
 * (scripts/generate/_generation.py:43). Here one token step keeps a KV cache, and the
 * work between two fused LoRA projections is one launch each. Conventions as in
 * wsl_lora.h: device pointers, bf16 tensors, explicit leading dimensions, work enqueued on
 * `stream`, return WSL_OK or a negative WSL_E_* code (wsl_decode_last_error() describes
 * the last failure of these entry points). Arithmetic is fp32 with one rounding to bf16
 * per output.
 *
 * KV cache layout (one layer): k_cache, v_cache [batch, n_kv_heads, cache_len, head_dim].
 * `pos` is a device int64 scalar (the position of the token being decoded), so a step can
 * be captured once in a HIP graph and replayed with pos advanced on the device.
 */
#ifndef WSL_DECODE_H
#define WSL_DECODE_H

#include <stddef.h>
#include <stdint.h>

#include "wsl_lora.h"

#ifdef __cplusplus
extern "C" {
#endif

/* h = x (+ residual, the sum rounded to bf16), written to h_out when it is not NULL;
 * out = h * rsqrt(mean(h^2) + eps) * weight.   x, residual, h_out, out [rows, dim], weight [dim].
 * Replaces RMSNorm (qwen3/model/model.py:296-314 attention_norm / ffn_norm / norm) and the
 * residual add before it. dim % 8 == 0, dim <= 8192; 16-byte aligned rows. */
int wsl_rmsnorm_fwd(const void* x, int64_t ldx, const void* residual, int64_t ldr, const void* weight,
                    float eps, void* out, int64_t ldo, void* h_out, int64_t ldh, int64_t rows, int64_t dim,
                    void* stream);

/* One decode token per sequence. qkv [batch, ldqkv] holds q | k | v heads
 * ([n_heads + 2 n_kv_heads] x head_dim). q and k are RMS-normed over head_dim
 * (q_norm_w / k_norm_w [head_dim]), rotated by RoPE row `*pos` of `rope`
 * ([*, 2 head_dim] fp32: cos then sin), q written to q_out [batch, n_heads, head_dim],
 * k and v written into the caches at position *pos. Replaces
 * qwen3/model/model.py:195-198 (q/k norm) and :73-90 (apply_rotary_emb) plus the cache
 * write. head_dim in {64, 128, 256}. */
int wsl_qk_norm_rope_fwd(const void* qkv, int64_t ldqkv, int64_t batch, int64_t n_heads, int64_t n_kv_heads,
                         int64_t head_dim, const void* q_norm_w, const void* k_norm_w, float eps,
                         const float* rope, const int64_t* pos, void* q_out, void* k_cache, void* v_cache,
                         int64_t cache_len, void* stream);

/* out [batch, n_heads * head_dim] = softmax(q . K^T * scale) . V over cache positions
 * 0..*pos, query head h reading kv head h / (n_heads / n_kv_heads). Replaces the
 * repeat_kv + scaled_dot_product_attention of qwen3/model/model.py:93-102,204-214 for one
 * query token. The cache length is split into 64-position chunks whose partial softmax
 * records go to `workspace` (wsl_decode_attention_workspace_bytes(...) bytes, 16-byte
 * aligned, contents irrelevant) and are merged by a second launch.
 * n_heads / n_kv_heads in {1, 2, 4, 8}; head_dim in {64, 128}. */
size_t wsl_decode_attention_workspace_bytes(int64_t batch, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                             int64_t cache_len);
int wsl_decode_attention_fwd(const void* q, const void* k_cache, const void* v_cache, int64_t batch,
                             int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t cache_len,
                             const int64_t* pos, float scale, void* out, void* workspace, size_t workspace_bytes,
                             void* stream);

/* One launch for the attention block of a decode step: wsl_qk_norm_rope_fwd's work (q and
 * k RMS-normed and rotated, k and v written into the caches at *pos) fused with
 * wsl_decode_attention_fwd's (out [batch, n_heads * head_dim]). Every 64-position chunk
 * workgroup normalises its own query heads; the chunk holding *pos also produces the step's
 * k and v. The chunks' partial softmax records are merged by the last one of each
 * (sequence, kv head) to finish. `workspace` (wsl_decode_attention_step_workspace_bytes
 * bytes, 256-byte aligned) starts with a fixed 64 KB region of arrival counters: zero-fill
 * it before its first use; every completed call, of any shape, leaves them zero. Calls
 * that may run concurrently must not share a workspace. n_heads / n_kv_heads in {1, 2, 4};
 * head_dim in {64, 128}; batch * n_kv_heads <= 16384. */
size_t wsl_decode_attention_step_workspace_bytes(int64_t batch, int64_t n_heads, int64_t n_kv_heads,
                                                  int64_t head_dim, int64_t cache_len);
int wsl_decode_attention_step_fwd(const void* qkv, int64_t ldqkv, int64_t batch, int64_t n_heads,
                                  int64_t n_kv_heads, int64_t head_dim, const void* q_norm_w, const void* k_norm_w,
                                  float eps, const float* rope, const int64_t* pos, void* k_cache, void* v_cache,
                                  int64_t cache_len, float scale, void* out, void* workspace, size_t workspace_bytes,
                                  void* stream);

/* out [rows, ffn] = silu(g) * u with g = gate_up[:, :ffn], u = gate_up[:, ffn:2 ffn].
 * Replaces F.silu(w1(x)) * w3(x) (qwen3/model/model.py:250-251) given the two projections'
 * outputs side by side. ffn % 8 == 0; 16-byte aligned rows. */
int wsl_swiglu_fwd(const void* gate_up, int64_t ld, int64_t rows, int64_t ffn, void* out, int64_t ldo,
                   void* stream);

/* out[row] = index of the largest x[row, 0..n) (bf16): the greedy token of a row of logits
 * (scripts/generate/_generation.py:26-29 with top_k = 1 keeps only the argmax). Ties give
 * the first index and NaN counts as largest, as torch.argmax. Rows that are 16-byte aligned
 * with ldx % 8 == 0 are read 16 bytes at a time.
 * With a workspace (wsl_argmax_rows_workspace_bytes bytes, 256-byte aligned, zero-filled
 * before its first use; every completed call leaves it zero; n < 2^32) each row is split
 * over up to 64 workgroups merged by a 64-bit atomic max; with workspace == NULL one
 * workgroup reads each row. */
size_t wsl_argmax_rows_workspace_bytes(int64_t rows, int64_t n);
int wsl_argmax_rows_fwd(const void* x, int64_t ldx, int64_t rows, int64_t n, int64_t* out, void* workspace,
                        size_t workspace_bytes, void* stream);

/* The fused LoRA linear of wsl_lora_linear_fwd (bf16 w, decode-shaped 1 <= M <= 64) with
 * the decode step's elementwise work folded into the same launch. `fuse` combines:
 *   WSL_FUSE_RMSNORM   the projection input is bf16(x * rsqrt(mean(x^2) + eps) * norm_w),
 *                      the block's pre-attention / pre-FFN RMSNorm
 *                      (qwen3/model/model.py:296-314, torch.nn.RMSNorm); norm_w [K] bf16;
 *   WSL_FUSE_SWIGLU    w and b hold the gate and up projections' rows interleaved in blocks
 *                      of 8 (rows 16j..16j+7 = gate rows 8j..8j+7, rows 16j+8..16j+15 = up
 *                      rows 8j..8j+7), a = [A_gate; A_up] with b's columns to match, and
 *                      y [M, N/2] = bf16(silu(gate) * up) (qwen3/model/model.py:250-251);
 *   WSL_FUSE_RESIDUAL  y = bf16(residual + bf16(projection)), the residual add h + attn(h)
 *                      or h + ffn(h) (qwen3/model/model.py:313-314); residual [M, ldr] bf16
 *                      may be y itself (each element is read before it is written).
 * SWIGLU and RESIDUAL exclude each other. M == 0 is a no-op. Errors, workspace and streams are those of
 * wsl_lora_linear_fwd (its workspace size query applies), reported by wsl_last_error().
 * Shapes the fused form does not cover return WSL_E_SHAPE; wsl_lora_linear_fused_supported
 * answers from the sizes alone (1 or 0, taking 16-byte aligned operands). */
#define WSL_FUSE_RMSNORM 1
#define WSL_FUSE_SWIGLU 2
#define WSL_FUSE_RESIDUAL 4
int wsl_lora_linear_fused_supported(int64_t M, int64_t N, int64_t K, int64_t r, int32_t fuse);
int wsl_lora_linear_fused_fwd(const void* x, int64_t ldx, const void* norm_w, float eps, const void* w,
                              int64_t ldw, const void* a, int64_t lda, const void* b, int64_t ldb, float scale,
                              const void* residual, int64_t ldr, void* y, int64_t ldy, int64_t M, int64_t N,
                              int64_t K, int64_t r, int32_t fuse, void* workspace, size_t workspace_bytes,
                              void* stream);

/* The tied output head fused with greedy sampling: out[m] = argmax_n bf16(x[m] . w[n]) for
 * x [M, K] and w [N, K] bf16 (the factorized head's second factor: x = h . P, w = E), in one
 * launch that streams w once and writes no logits. Replaces the head matmul and the
 * argmax of scripts/generate/_generation.py:19-32 (top_k = 1 keeps only the argmax) over
 * the tied output (torchtitan/experiments/qwen3/infra/parallelize.py:123-125); the result is
 * torch.argmax of the bf16 logits the unfused head stores (ties give the first index, NaN
 * counts as largest). out [M] int64. 1 <= M <= 64, N < 2^32, and a short K (two wave steps
 * of 128, e.g. the rank-256 factor); wsl_tied_head_argmax_supported answers from the sizes
 * alone (16-byte aligned operands). The workspace (wsl_tied_head_argmax_workspace_bytes(M)
 * bytes, 256-byte aligned) is zero-filled before its first use; every completed call
 * leaves it valid for the next. Errors are reported by wsl_last_error(). */
size_t wsl_tied_head_argmax_workspace_bytes(int64_t M);
int wsl_tied_head_argmax_supported(int64_t M, int64_t N, int64_t K);
int wsl_tied_head_argmax_fwd(const void* x, int64_t ldx, const void* w, int64_t ldw, int64_t N, int64_t K, int64_t M,
                             int64_t* out, void* workspace, size_t workspace_bytes, void* stream);

/* A chain of decode-shaped LoRA linears in one persistent launch. No counterpart in the
 * reference, whose decode re-runs the whole model per token (scripts/generate/_generation.py:35-80)
 * with one aten call per projection; it replaces the consecutive launches of the projections
 * of one decode step (torchtitan/experiments/qwen3/model/model.py:184,218,250-251 at M tokens).
 *
 * Stage s is wsl_lora_linear_fused_fwd (fuse != 0) or wsl_lora_linear_grouped_fwd (fuse == 0,
 * n_groups >= 1) on its descriptor, with the same results bit for bit. One workgroup per CU
 * runs every stage's workgroups in order; a stage with after_previous = 1 reads what an
 * earlier stage of the chain wrote (its x or residual), so its workgroups wait until every
 * workgroup of the previous stage has stored its outputs. They issue their first W and A
 * loads before that wait and fetch x afterwards, so a stage's weight stream overlaps the end
 * of the stage before it. Stages without after_previous must not read another stage's output.
 *
 * Shapes taken (wsl_lora_linear_chain_supported, from the sizes and pointer alignment):
 * 1 <= M <= 16, bf16 W, 1 <= n_stages <= WSL_CHAIN_MAX_STAGES; each stage the decode path's
 * one-slice plan (x, A and B rows in one K slice: M * K * 2 bytes within the LDS budget; K a
 * multiple of 128 and at least 1024), N a multiple of 16 and at most 1024 output row blocks
 * (16 or 32 rows each, 16384 rows at least), 16-byte aligned operands. Errors are reported
 * by wsl_last_error().
 *
 * Waits are bounded. A stage wait that gives up sets a sticky failure word in the workspace
 * and the launch still drains (its outputs are then not valid);
 * wsl_lora_linear_chain_status reads and clears that word (it synchronizes `stream`). The
 * workspace (wsl_lora_linear_chain_workspace_bytes) is zero-filled before its first use and
 * kept valid by every call; a workspace used only by chains keeps other launches' hand-off
 * words out of the chain's stage flags. */
#define WSL_CHAIN_MAX_STAGES 8
typedef struct wsl_chain_stage {
  const void* x; int64_t ldx;    /* input [M, K] bf16 */
  const void* norm_w; float eps; /* RMSNorm weight [K] (fuse & WSL_FUSE_RMSNORM) */
  const void* w; int64_t ldw;    /* base [N, K] bf16 */
  const void* a; int64_t lda;    /* LoRA A [n_groups * r, K] (r = 0: none) */
  const void* b; int64_t ldb;    /* LoRA B [N, r] */
  float scale;
  const void* residual; int64_t ldr; /* fuse & WSL_FUSE_RESIDUAL */
  void* y; int64_t ldy;          /* output [M, N], or [M, N / 2] with WSL_FUSE_SWIGLU */
  int64_t N, K, r;
  int32_t fuse;                  /* WSL_FUSE_* as wsl_lora_linear_fused_fwd, or 0 */
  int32_t n_groups;              /* fuse == 0: projections side by side (group_n), else 1 */
  int64_t group_n[4];
  int32_t after_previous;        /* 1: x or residual is an earlier stage's output */
} wsl_chain_stage;
int wsl_lora_linear_chain_supported(int64_t M, int32_t n_stages, const wsl_chain_stage* stages);
int wsl_lora_linear_chain_workspace_bytes(int64_t M, int32_t n_stages, const wsl_chain_stage* stages,
                                          size_t* bytes);
int wsl_lora_linear_chain_fwd(int64_t M, int32_t n_stages, const wsl_chain_stage* stages, void* workspace,
                              size_t workspace_bytes, void* stream);
int wsl_lora_linear_chain_status(void* workspace, void* stream, int32_t* failed);

/* Thread-local description of the last failure of an entry point above ("" if none). */
const char* wsl_decode_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* WSL_DECODE_H */
