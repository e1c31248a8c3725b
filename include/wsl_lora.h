/*
 * wsl_lora.h — C ABI of the MI355X (gfx950) fused LoRA linear library (libwsl.so).
 *
 * The reference (muchanem/weightshared_torchtitan) has no native boundary for this
 * path: the LoRA linear is three nn.Linear calls plus a mul and an add inside
 * Attention.forward. Each entry point below names the reference code it replaces.
 *
 * Conventions shared by every entry point:
 *   - Row-major matrices with an explicit leading dimension (elements between rows);
 *     the inner dimension is contiguous. Shapes follow nn.Linear: y = x . W^T.
 *   - The caller owns every buffer. Nothing here allocates or frees device memory;
 *     scratch space is passed in (see wsl_lora_linear_workspace_bytes).
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the default stream) and is
 *     stream-ordered. No entry point synchronizes the host.
 *   - Return value: WSL_OK (0) or a negative WSL_E_* code. Nothing throws across the
 *     ABI. wsl_last_error() returns a thread-local description of the last failure.
 *   - bf16 is bfloat16 (1-8-7); fp8 is OCP float8_e4m3fn (bias 7, max 448, no inf).
 */
#ifndef WSL_LORA_H
#define WSL_LORA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WSL_OK 0
#define WSL_E_INVALID_ARG (-1) /* null pointer where one is required, bad enum   */
#define WSL_E_SHAPE (-2)       /* negative / inconsistent sizes or leading dims   */
#define WSL_E_DTYPE (-3)       /* unsupported w_dtype                             */
#define WSL_E_ALIGN (-4)       /* pointer or leading dimension misaligned         */
#define WSL_E_WORKSPACE (-5)   /* workspace missing or smaller than required      */
#define WSL_E_DEVICE (-6)      /* no HIP device, or device is not gfx950          */
#define WSL_E_LAUNCH (-7)      /* a kernel launch failed                          */

/* Storage type of the base weight W.
 *   WSL_DTYPE_FP8_E4M3       fp8 W with per-output-channel fp32 scales; the activations keep
 *                            bf16 precision: on prefill shapes (M > 64) the product runs on
 *                            the fp8 matrix cores with each activation split into two e4m3
 *                            terms under a per-token power-of-two scale (x = 2^e (hi + lo/16),
 *                            exact to 2^-8), on decode shapes W is decoded to bf16.
 *   WSL_DTYPE_FP8_E4M3_ACT8  the same weight, with the prefill product on one e4m3 term per
 *                            activation: half the matrix-core work, plus e4m3 rounding of x
 *                            (about 3.7e-2 against an fp32-W reference at config-5 shapes,
 *                            against 2.4-2.6e-2 for WSL_DTYPE_FP8_E4M3). Decode shapes as above. */
#define WSL_DTYPE_BF16 0
#define WSL_DTYPE_FP8_E4M3 1
#define WSL_DTYPE_FP8_E4M3_ACT8 2

/* Largest LoRA rank the kernels accept. */
#define WSL_MAX_RANK 256

/*
 * Bytes of scratch memory wsl_lora_linear_fwd needs for this problem. Pure host
 * function: touches no device.
 *
 * Workspace contract: the workspace must be zero-filled before its first use. It
 * starts with WSL_COUNTER_BYTES holding a launch counter (the rest of the prefix stays
 * zero) that every completed call leaves valid for the next one, so a workspace is
 * allocated and zeroed once and then reused; do not modify it between calls. Calls that
 * may run concurrently (different streams) must not share a workspace. The rest of the
 * workspace holds scratch data and launch-tagged hand-off words.
 */
#define WSL_COUNTER_BYTES 65536
int wsl_lora_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r,
                                    int32_t w_dtype, size_t* bytes);

/*
 * Fused LoRA linear:  y[M,N] = (x . W^T) * diag(w_scale) + scale * (x . A^T) . B^T
 *
 * Replaces, for one projection, the reference's
 *   base  = nn.Linear(K, N)(x)                       torchtitan/models/llama3/model/model.py:257-273,392-394
 *   delta = w_b(w_a(x)) * (alpha / rank)             torchtitan/models/llama3/model/model.py:189-192
 *   y     = broadcast_add(base, delta)  (g = 1 case) torchtitan/models/llama3/model/model.py:111-145,396-398
 *
 *   x        [M,K] bf16, row stride ldx.
 *   w        [N,K] bf16 (w_dtype = WSL_DTYPE_BF16) or fp8 e4m3fn (WSL_DTYPE_FP8_E4M3),
 *            row stride ldw. May be NULL: then y is the LoRA delta alone (the
 *            reference LoRAModule.forward).
 *   w_scale  [N] fp32 per-output-channel dequantisation scale. Required for fp8,
 *            must be NULL for bf16.
 *   a        [r,K] bf16 (LoRAModule.w_a.weight), row stride lda.
 *   b        [N,r] bf16 (LoRAModule.w_b.weight), row stride ldb.
 *            r = 0 (a, b ignored) gives the plain linear.
 *   scale    LoRA scale s = alpha / rank (2.0 under the reference's alpha = 2*rank).
 *   y        [M,N] bf16 output, row stride ldy. Must not alias any input.
 *   Accumulation is fp32. x . A^T is rounded once to bf16 after scaling by s.
 *   M may be 0 (no work). K >= 1, N >= 1, 0 <= r <= WSL_MAX_RANK.
 */
int wsl_lora_linear_fwd(const void* x, int64_t ldx,
                        const void* w, int64_t ldw, int32_t w_dtype, const float* w_scale,
                        const void* a, int64_t lda,
                        const void* b, int64_t ldb,
                        float scale,
                        void* y, int64_t ldy,
                        int64_t M, int64_t N, int64_t K, int64_t r,
                        void* workspace, size_t workspace_bytes,
                        void* stream);

/*
 * wsl_lora_linear_fwd without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It has no counterpart in the reference. Same arguments, results and errors as
 * wsl_lora_linear_fwd (the same kernels run); the scratch memory lives in a static device
 * array of WSL_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends. A problem whose
 * scratch need exceeds it returns WSL_E_WORKSPACE before touching a device. Nothing here
 * allocates or frees memory.
 *   - The first call on a device sets the array up (its address, a zero fill on `stream`
 *     and a synchronisation of `stream`); that call may not be under graph capture
 *     (WSL_E_INVALID_ARG). Later calls may be captured.
 *   - Every call on a GPU shares that GPU's array: calls that may overlap on one GPU (on
 *     different streams without ordering between them) race and must not be issued.
 */
#define WSL_NOALLOC_SCRATCH_BYTES (64 * 1024 * 1024)
int wsl_lora_linear_fwd_noalloc(const void* x, int64_t ldx,
                                const void* w, int64_t ldw, int32_t w_dtype, const float* w_scale,
                                const void* a, int64_t lda,
                                const void* b, int64_t ldb,
                                float scale,
                                void* y, int64_t ldy,
                                int64_t M, int64_t N, int64_t K, int64_t r,
                                void* stream);

/*
 * Grouped fused LoRA linear: up to WSL_MAX_GROUPS projections that read the same x, in
 * one call. Group g covers output columns [n_g, n_g + group_n[g]) with
 * n_g = group_n[0] + ... + group_n[g-1], and
 *
 *   y[:, n_g : n_g + group_n[g]] = x . W_g^T (* diag(w_scale_g)) + scale * (x . A_g^T) . B_g^T
 *
 * which is exactly wsl_lora_linear_fwd on each group's column range. Operands are the
 * groups' tensors stacked: w [N,K] (W_g rows stacked, N = sum of group_n), w_scale [N],
 * b [N,r] (B_g rows stacked), y [N columns], and a [n_groups*r, K] (A_g is rows
 * g*r .. g*r+r-1). Every group has rank r. group_n is a host array.
 *
 * Replaces the projections of one reference block that read the same activation: q, k
 * and v (torchtitan/models/llama3/model/model.py:376-398, each base + broadcast_add of
 * its LoRA delta; Qwen3 wq/wk/wv, torchtitan/experiments/qwen3/model/model.py:184) and
 * gate/up (qwen3/model/model.py:250-251). The groups run as one launch where every group
 * boundary falls on the launch's work grid: on the prefill path, whole output tiles
 * (multiples of 128; of 256 for ranks 33-64), each tile taking its group's rank block; on
 * the decode path (M <= 64; plain bf16 up to 72 with WSL_OPT_DECODE_WIDE), whole row groups of W (multiples of 64
 * suffice), the T work covering all groups' A rows. Otherwise the groups run as consecutive
 * launches on `stream`. Results are those of the per-group calls, bit for bit, except where
 * a K split count depends on N (the decode path's wide form; the prefill
 * path's in-launch split-K form, taken where 128 x 128 tiles leave CUs idle), where the
 * column tiles of a launch share T (WSL_OPT_PREFILL_SHARED_T; one wave of tiles), where T
 * comes from the rank pre-pass (ranks above 64, and ranks 33-64 where it frees a tile wider
 * than 128 x 128, which depends on N; its K split count follows all groups' ranks) or, for an
 * fp8 W on prefill shapes, where the choice between the fp8 matrix cores and W decoded onto
 * the bf16 matrix cores depends on the launch's width (WSL_OPT_FP8_PREFILL): there the
 * groups' outputs agree with the per-group calls within the forward's bar.
 */
#define WSL_MAX_GROUPS 4
int wsl_lora_linear_grouped_workspace_bytes(int64_t M, int64_t K, int64_t r, int32_t n_groups,
                                            const int64_t* group_n, int32_t w_dtype, size_t* bytes);
int wsl_lora_linear_grouped_fwd(const void* x, int64_t ldx,
                                const void* w, int64_t ldw, int32_t w_dtype, const float* w_scale,
                                const void* a, int64_t lda,
                                const void* b, int64_t ldb,
                                float scale,
                                void* y, int64_t ldy,
                                int64_t M, int64_t K, int64_t r,
                                int32_t n_groups, const int64_t* group_n,
                                void* workspace, size_t workspace_bytes,
                                void* stream);

/*
 * Shared-base LoRA linears: one base weight W [base_n, K] serving n_groups projections, each
 * with its own LoRA factors, and optionally shared across head groups:
 *
 *   y[:, j N : (j + 1) N] = broadcast_add(x . W^T (* w_scale), scale * (x . A_j^T) . B_j^T, g)
 *
 * with broadcast_add as the reference's (torchtitan/models/llama3/model/model.py:111-145):
 * output column c of a group reads base column (c / (hpg D')) D' + c % D', D' = base_n / g,
 * hpg = N / base_n. Replaces the reference's attention compositions
 *   head_sharing: xq = broadcast_add(wq_base(x), wq_offset(x), g = grouping)  (model.py:255-273,
 *                 396-398; base_n = grouping * head_dim < N), and
 *   qkv_sharing:  one base module for q, k and v, val = base(x) added to each projection's
 *                 offset (model.py:239-253, 381-398; n_groups = 3, base_n = N),
 * in one launch that never materialises the expanded base: every kernel reads W rows through
 * the column map. a [n_groups * r, K] (A_j = rows j r .. j r + r - 1), b [n_groups * N, r],
 * y [M, n_groups * N] columns, w_scale [base_n] (fp8 W). N % base_n == 0, base_n % g == 0,
 * 1 <= n_groups <= WSL_MAX_GROUPS. Workspace from wsl_lora_linear_bcast_workspace_bytes.
 */
int wsl_lora_linear_bcast_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, int32_t n_groups,
                                          int32_t w_dtype, size_t* bytes);
int wsl_lora_linear_bcast_fwd(const void* x, int64_t ldx,
                              const void* w, int64_t ldw, int32_t w_dtype, const float* w_scale,
                              const void* a, int64_t lda,
                              const void* b, int64_t ldb,
                              float scale,
                              void* y, int64_t ldy,
                              int64_t M, int64_t N, int64_t K, int64_t r,
                              int64_t base_n, int64_t g, int32_t n_groups,
                              void* workspace, size_t workspace_bytes,
                              void* stream);

/*
 * Weight gradients of y = x . W^T + scale * (x . a^T) . b^T, given gy = dL/dy:
 *
 *   dw = gy^T . x                  [N, K]   (row stride lddw)
 *   da = scale * (gy . b)^T . x    [r, K]   (row stride ldda)
 *   db = scale * gy^T . (x . a^T)  [N, r]   (row stride lddb)
 *
 * (scale * gy . b and scale * x . a^T are rounded to bf16 once, as the forward's rank
 * pre-pass rounds its T.) Replaces what torch autograd computes for the reference's
 * LoRAModule.forward (torchtitan/models/llama3/model/model.py:189-192) and the base
 * nn.Linear (:257-273) composed by broadcast_add (:392-398), as run by the trainer's
 * loss.backward() (torchtitan/train.py:456); the reference has no kernel of its own.
 * All tensors bf16 [rows, ld]; x [M, K], gy [M, N], a [r, K], b [N, r]. Any of dw, da, db
 * may be NULL (not computed); da and db need r > 0. Deterministic: split reductions are
 * summed in a fixed order. wsl_lora_linear_bwd_weights_supported returns 1 for the layouts
 * the MFMA tile kernels take (K and N multiples of 64, r a multiple of 8, x, gy, a, b 16-byte
 * aligned with leading dimensions multiples of 8) and 0 for the rest, which run on scalar
 * kernels with the same contract (dW, dB = gy^T . T and dA = U^T . x over the tokens).
 * Workspace (256-byte aligned) from wsl_lora_linear_bwd_weights_workspace_bytes; it may be
 * the forward's workspace (the decode path's counter prefix is left as it is).
 */
int wsl_lora_linear_bwd_weights_supported(const void* x, int64_t ldx, const void* gy, int64_t ldg,
                                          const void* a, int64_t lda, const void* b, int64_t ldb,
                                          int64_t M, int64_t N, int64_t K, int64_t r);
int wsl_lora_linear_bwd_weights_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, size_t* bytes);
int wsl_lora_linear_bwd_weights(const void* x, int64_t ldx, const void* gy, int64_t ldg,
                                const void* a, int64_t lda, const void* b, int64_t ldb,
                                float scale, int64_t M, int64_t N, int64_t K, int64_t r,
                                void* dw, int64_t lddw, void* da, int64_t ldda, void* db, int64_t lddb,
                                void* workspace, size_t workspace_bytes,
                                void* stream);

/*
 * Input gradient of the fused LoRA linear:
 *
 *   dx [M, K] = gy [M, N] . W [N, K] (. diag(w_scale) folded per row of W) + scale * (gy . B) . A
 *
 * with W [N, K] (bf16, or e4m3 with w_scale [N] fp32: WSL_DTYPE_FP8_E4M3 or _ACT8), A [r, K],
 * B [N, r] the operands as wsl_lora_linear_fwd takes them: W is read where it lies (no
 * transposed copy), as the reduction rows of the fused kernel's token-major W tiles; an fp8
 * W is decoded to bf16(code * w_scale[n]) as its tiles are staged (the dequantised W). Replaces the dx half of torch autograd's backward of the reference's
 * LoRA linear (LoRAModule.forward, torchtitan/models/llama3/model/model.py:189-192, plus
 * the base nn.Linear, :257-273), run by loss.backward() (torchtitan/train.py:456).
 * wsl_lora_linear_bwd_input_supported returns 1 for the layouts taken: N a multiple of 64,
 * K and r multiples of 8 (K of 16 for fp8), r <= WSL_MAX_RANK, gy, W, A, B and dx 16-byte
 * aligned with leading dimensions multiples of 8 (fp8 ldw of 16; dx: 8-byte aligned, ldd a
 * multiple of 4); the rest return WSL_E_SHAPE (or WSL_E_ALIGN), and a caller multiplies by
 * a transposed copy of W instead.
 * Workspace (256-byte aligned) from wsl_lora_linear_bwd_input_workspace_bytes: the forward's
 * prefill scratch for [M, K] outputs plus the transposed A and B. fp32 accumulation, T =
 * bf16(scale * gy . B) rounded once, as the forward.
 */
int wsl_lora_linear_bwd_input_supported(const void* gy, int64_t ldg, const void* w, int64_t ldw, int32_t w_dtype,
                                        const float* w_scale, const void* a, int64_t lda, const void* b, int64_t ldb,
                                        const void* dx, int64_t lddx, int64_t M, int64_t N, int64_t K, int64_t r);
int wsl_lora_linear_bwd_input_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, size_t* bytes);
int wsl_lora_linear_bwd_input(const void* gy, int64_t ldg, const void* w, int64_t ldw, int32_t w_dtype,
                              const float* w_scale, const void* a, int64_t lda, const void* b, int64_t ldb,
                              float scale, void* dx, int64_t lddx,
                              int64_t M, int64_t N, int64_t K, int64_t r,
                              void* workspace, size_t workspace_bytes, void* stream);

/*
 * Factorized embedding:  out[t, :] = E[ids[t], :] . P^T      (k -> hidden)
 *
 * Replaces the reference's token embedding nn.Embedding(vocab, dim)
 * (torchtitan/models/llama3/model/model.py:561, torchtitan/experiments/qwen3/model/model.py:350)
 * with a rank-k factorisation: E [vocab,k] bf16 (row stride lde), P [hidden,k] bf16
 * (row stride ldp, nn.Linear(k, hidden).weight layout). out [n_ids, hidden] bf16,
 * row stride ldo. ids are int64; an id outside [0, vocab) sets that row to zero
 * (the kernel never reads out of bounds). k <= 1024.
 */
int wsl_factorized_embedding_fwd(const int64_t* ids, int64_t n_ids,
                                 const void* emb, int64_t lde, int64_t vocab, int64_t k,
                                 const void* proj, int64_t ldp, int64_t hidden,
                                 void* out, int64_t ldo,
                                 void* stream);

/*
 * Path overrides. No counterpart in the reference (whose path is three aten calls with no
 * choices to make); they exist for side-by-side timing and for tests that pin one form of a
 * kernel against the oracle. Each option is a process-wide integer that starts at 0, the
 * library's own choice; the host planning of every later launch reads it. Set them between
 * calls, never while another thread is launching. Every form computes the same contract
 * within the forward's bar; the ones marked bit-exact give identical outputs.
 *   WSL_OPT_PREFILL_STRIPS     0 auto; -1 one output tile per workgroup (bit-exact)
 *   WSL_OPT_PREFILL_SPLIT      0 auto; -1 never split K inside a launch; n in [2, 16] that
 *                              split count wherever it divides the K tiles and fits
 *   WSL_OPT_PREFILL_MEDIUM     0 auto; -1 never take the medium-M split form
 *   WSL_OPT_FP8_PREFILL        0 auto (two activation terms on the fp8 matrix cores where
 *                              the launch has more 256 x 256 tiles than CUs, else W decoded
 *                              onto the bf16 matrix cores); 1 always decoded; 2 always the
 *                              fp8 matrix cores
 *   WSL_OPT_DECODE_PASSES      0 auto; -1 K splits only; 1 passes wherever the slices allow
 *   WSL_OPT_DECODE_WIDE        0 or -1: 65-72 tokens on the prefill path (the default); 1 the
 *                              decode path's wide form for plain bf16 launches of 65-72 tokens
 *   WSL_OPT_DECODE_SPIN_LIMIT  0 the default poll bound of the decode hand-offs; n > 0 that
 *                              bound; -1 no polling (the local fallback runs at once)
 *   WSL_OPT_DECODE_RES_SPLITS  0 auto; n in [2, 8] at least n K splits for the decode step's
 *                              residual-epilogue launches (wsl_lora_linear_fused_fwd) where
 *                              the slices keep eight wave steps
 *   WSL_OPT_PREFILL_SHARED_T   0 auto (one-wave launches of one in-loop rank block over
 *                              K >= 4096 share T between the column tiles of each row
 *                              block); -1 T in every
 *                              tile; 1 shared, with every tile taking the no-wait path (it
 *                              computes the classes of T from global memory: bit-exact
 *                              with 0); 2 shared at any K (one-wave launches)
 * wsl_set_option returns WSL_E_INVALID_ARG for an unknown option or a value out of range.
 */
#define WSL_OPT_PREFILL_STRIPS 1
#define WSL_OPT_PREFILL_SPLIT 2
#define WSL_OPT_PREFILL_MEDIUM 3
#define WSL_OPT_FP8_PREFILL 4
#define WSL_OPT_DECODE_PASSES 5
#define WSL_OPT_DECODE_WIDE 6
#define WSL_OPT_DECODE_SPIN_LIMIT 7
#define WSL_OPT_DECODE_RES_SPLITS 8
#define WSL_OPT_PREFILL_SHARED_T 9
#define WSL_OPT_COUNT 10
int wsl_set_option(int32_t option, int64_t value);
int wsl_get_option(int32_t option, int64_t* value);

/*
 * The plan a grouped (n_groups >= 1) or single call of these sizes takes, for dense,
 * 256-byte aligned operands (pointer alignment also steers the path). No counterpart in the
 * reference; it lets tests assert which kernel form their shapes reach. Host function: it
 * launches nothing (shared_t reads the current device's CU count; 0 without a device).
 *   path         WSL_PATH_*; WSL_PATH_NONE for M = 0
 *   launches     calls of the main kernel (a grouped call that cannot run as one launch
 *                runs group by group: n_groups)
 *   tile_m/n     output tile of one workgroup on the prefill paths (of the first group's
 *                launch when the groups run one by one), else 0
 *   rank_blocks  32-rank blocks of T computed inside the K loop (0: none, or pre-pass T)
 *   rank_prepass 1 when T comes from the rank pre-pass launch
 *   strip_tiles  output tiles per workgroup of the persistent strips (1: one per workgroup)
 *   k_splits     K splits of the split-K forms (1 otherwise)
 *   workgroups   workgroups of the main launch on the prefill paths (first group's), else 0
 *   shared_t     1 when the column tiles of each row block share T (a launch of one wave of
 *                tiles on this device over K >= 4096: each group's first four tiles compute
 *                one class of T's k steps each, the other tiles none)
 */
#define WSL_PATH_NONE 0
#define WSL_PATH_PREFILL 1
#define WSL_PATH_PREFILL_SPLITK 2
#define WSL_PATH_PREFILL_MEDIUM 3
#define WSL_PATH_PREFILL_FP8 4
#define WSL_PATH_DECODE 5
#define WSL_PATH_GENERIC 6
typedef struct wsl_plan_info {
  int32_t path;
  int32_t launches;
  int32_t tile_m, tile_n;
  int32_t rank_blocks;
  int32_t rank_prepass;
  int32_t strip_tiles;
  int32_t k_splits;
  int32_t workgroups;
  int32_t shared_t;
} wsl_plan_info;
int wsl_lora_linear_plan(int64_t M, int64_t K, int64_t r, int32_t n_groups, const int64_t* group_n,
                         int32_t w_dtype, wsl_plan_info* out);

/* Thread-local, NUL-terminated description of the last error ("" if none). */
const char* wsl_last_error(void);

/* Library ABI version (major * 100 + minor). */
int wsl_version(void);

#ifdef __cplusplus
}
#endif

#endif /* WSL_LORA_H */
