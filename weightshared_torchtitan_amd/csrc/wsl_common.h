// Shared device-side types and helpers for the gfx950 kernels of libwsl.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wsl_lora.h"

namespace wsl {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;

// Storage type tags (match WSL_DTYPE_* in include/wsl_lora.h).
enum : int { kBF16 = 0, kFP8 = 1 };

// Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16 bits, round to nearest even, NaN kept NaN with its quiet bit set. Lowers to
// gfx950's v_cvt_pk_bf16_f32, which matches the integer rounding u + 0x7fff + ((u >> 16) & 1)
// (and (u >> 16) | 0x40 for NaN) on all 2^32 inputs; the branch of the integer form for NaN
// costs exec-mask juggling per element in the epilogues.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// fp32 rounded to the nearest bf16 value.
__device__ __forceinline__ float bf16_round(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// Two fp32 -> packed bf16x2 (low half = a).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// Four OCP e4m3fn bytes (packed in one dword, byte 0 first) -> 4 bf16 in two dwords.
// gfx950's v_cvt_pk_f32_fp8 decodes the OCP format; every e4m3fn value is exactly
// representable in bf16, so truncating the fp32 result is exact.
template <bool HIGH_HALF>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t q) {
  auto f = __builtin_amdgcn_cvt_pk_f32_fp8((int)q, HIGH_HALF);
  return (__float_as_uint(f[0]) >> 16) | (__float_as_uint(f[1]) & 0xffff0000u);
}

// 16 fp8 (one 16-byte chunk) -> 16 bf16 (two 16-byte chunks).
__device__ __forceinline__ void fp8x16_to_bf16x16(const u32x4_t& q, u32x4_t& lo, u32x4_t& hi) {
  lo = u32x4_t{fp8x2_to_bf16x2<false>(q[0]), fp8x2_to_bf16x2<true>(q[0]),
               fp8x2_to_bf16x2<false>(q[1]), fp8x2_to_bf16x2<true>(q[1])};
  hi = u32x4_t{fp8x2_to_bf16x2<false>(q[2]), fp8x2_to_bf16x2<true>(q[2]),
               fp8x2_to_bf16x2<false>(q[3]), fp8x2_to_bf16x2<true>(q[3])};
}

// 8 fp8 (two dwords) -> 8 bf16 (one 16-byte chunk).
__device__ __forceinline__ u32x4_t fp8x8_to_bf16x8(uint32_t q0, uint32_t q1) {
  return u32x4_t{fp8x2_to_bf16x2<false>(q0), fp8x2_to_bf16x2<true>(q0),
                 fp8x2_to_bf16x2<false>(q1), fp8x2_to_bf16x2<true>(q1)};
}

// Greedy-token key of (value, index): the value's order-preserving bits (NaN above
// everything, -0 folded into +0) over the complemented index, so the larger key is the
// larger value and, among equal values, the lower index (torch.argmax's order). Every key
// of a real value is above zero, so a zero word is "no candidate yet".
__device__ __forceinline__ uint64_t am_key(float v, int64_t i) {
  uint32_t o;
  if (v != v) {
    o = 0xffffffffu;
  } else {
    const uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);
    o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  }
  return ((uint64_t)o << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
}

// The index a key holds.
__device__ __forceinline__ int64_t am_index(uint64_t k) { return (int64_t)(0xffffffffu - (uint32_t)k); }

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ u32x4_t ld_global_16(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

__device__ __forceinline__ u32x4_t zero_u32x4() {
  u32x4_t z = {0u, 0u, 0u, 0u};
  return z;
}

}  // namespace wsl

// Host-side launch helpers shared by the translation units of libwsl.
namespace wsl {

// Base-row map of the shared-base forms (the reference's broadcast_add with g > 1, and one
// base weight serving several projections): output column c takes row
// ((c mod P) / S) * D + (c mod P) mod D of W and of w_scale. P == 0 is the identity.
// Every kernel maps the rows it reads once per tile or wave (never inside the K loop).
struct RowMap {
  int P = 0, S = 1, D = 1;
};
__host__ __device__ __forceinline__ int map_row(int c, const RowMap& m) {
  if (m.P == 0) return c;
  const int c2 = c % m.P;
  return (c2 / m.S) * m.D + c2 % m.D;
}

constexpr int kMaxGroups = 4;  // projections in one grouped launch (WSL_MAX_GROUPS)

struct LoraArgs {
  const void* x; int64_t ldx;
  const void* w; int64_t ldw; int w_dtype; const float* w_scale;
  const void* a; int64_t lda;
  const void* b; int64_t ldb;
  float scale;
  void* y; int64_t ldy;
  int64_t M, N, K, r;
  void* ws; size_t ws_bytes;
  hipStream_t stream;
  // Optional row gather on x: row m of x is row gather[m] of a [gather_rows, ldx] table;
  // ids outside [0, gather_rows) read as zero rows. Used by the factorized embedding.
  const int64_t* gather; int64_t gather_rows;
  // Factor applied to the fp32 result before the bf16 rounding of y (prefill path; the
  // rank pre-pass uses it to store bf16(s * x . A^T)).
  float yscale = 1.f;
  // Grouped launch (prefill path): `groups` projections side by side in N. Group g holds
  // output columns [gend[g-1], gend[g]) (gend[groups-1] = N) and uses rows g*r..g*r+r-1
  // of a; w, w_scale, b and y are indexed by the output column as usual.
  int groups = 1;
  int64_t gend[kMaxGroups] = {0, 0, 0, 0};
  // fp8 W on prefill shapes: activation terms of the fp8 matrix-core path (2: bf16-quality
  // activations, 1: one e4m3 term); 0 decodes W to bf16 on the bf16 matrix cores instead.
  int fp8_terms = 2;
  // Shared-base forms: W (and w_scale) rows by output column, and W's row count.
  RowMap wmap;
  int64_t wrows = 0;
  // Arrival counters of the prefill path's in-launch split-K form (the workspace prefix
  // from kRedCntOff); nullptr keeps that form off.
  unsigned* red_cnt = nullptr;
};

// Path overrides (WSL_OPT_* of include/wsl_lora.h): 0 unless wsl_set_option changed them.
int64_t option(int id);

// Compute units of the current device (cached per device; 0 when it cannot be read).
int device_cus();

// The prefill path's choice for a call (csrc/lora_prefill.hip), shared by the launcher and
// wsl_lora_linear_plan: form (WSL_PATH_PREFILL*), tile, in-loop rank blocks, pre-pass T,
// persistent strip length, K splits and the main launch's workgroups.
struct PrefillPlan {
  int form = 0;
  int tile_m = 0, tile_n = 0;
  int rank_blocks = 0;
  bool prepass = false;
  int strips = 1;
  int splits = 1;
  int64_t workgroups = 0;
  bool shared_t = false;
};
PrefillPlan plan_prefill(const LoraArgs& p);

// Each launcher returns hipSuccess or the launch error.
hipError_t launch_prefill(const LoraArgs& p);
size_t prefill_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, int w_dtype);
bool prefill_supported(const LoraArgs& p);
bool prefill_groups_supported(const LoraArgs& p);
// Whether every group end of a grouped launch falls on a multiple of bn columns.
bool groups_fit_tiles(const LoraArgs& p, int bn);
// K splits of the medium-M split form of the prefill path (0: not taken); rt = r * groups.
int medium_splits(int64_t M, int64_t N, int64_t K, int64_t rt, int w_dtype, bool has_w, bool gather);
// K splits of the prefill path's in-launch split-K form over 128 x 128 tiles (0: not taken;
// it also needs a rank of at most 64 per group).
int red_splits(int64_t M, int64_t N, int64_t K, int w_dtype, bool has_w, bool gather);
// Plain bf16 products over a long contiguous K (csrc/lora_prefill.hip) and the rank
// pre-pass T = bf16(s x . A^T), for the weight gradients (csrc/lora_backward.hip).
int product_splits(int64_t M, int64_t N, int64_t nk, bool divides);
hipError_t launch_product(const LoraArgs& p, float* part, int splits);
hipError_t launch_product_tn(const LoraArgs& p, int64_t tokens, float* part, int splits);
size_t rank_prepass_bytes(int64_t M, int64_t K, int64_t rt);
hipError_t rank_prepass(const LoraArgs& p, uint16_t* t);
// Weight gradients dW = gy^T x, dA = s (gy B)^T x, dB = s gy^T (x A^T) (csrc/lora_backward.hip).
bool weight_grads_supported(const LoraArgs& p, const void* gy, int64_t ldg);
size_t weight_grads_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, bool need_w, bool need_ab);
hipError_t launch_weight_grads(const LoraArgs& p, const void* gy, int64_t ldg, void* dw, int64_t lddw, void* da,
                               int64_t ldda, void* db, int64_t lddb);
// The input gradient dX = dY . W + s (dY . B) . A with W [N, K] read where it lies: the
// prefill kernel's WT form on the forward-shaped problem q (x = dY, K' = N, N' = K, a = B^T,
// b = A^T; csrc/lora_prefill.hip), and its driver from the linear's own operands (p: x =
// dY [M, N], w = W [N, K], a = A [r, K], b = B [N, r], y = dX [M, K]; p.N and p.K are the
// linear's), which transposes A and B into the workspace (csrc/lora_backward.hip).
bool prefill_wt_supported(const LoraArgs& q);
hipError_t launch_prefill_wt(const LoraArgs& q);
bool bwd_input_supported(const LoraArgs& p);
size_t bwd_input_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r);
hipError_t launch_bwd_input(const LoraArgs& p);

// fp8 matrix-core prefill path (csrc/lora_prefill_fp8.hip): T from the rank pre-pass, the
// activation codes and per-token scales in `scratch` (prefill_fp8_workspace_bytes).
bool prefill_fp8_supported(const LoraArgs& p);
size_t prefill_fp8_workspace_bytes(int64_t M, int64_t K, int terms);
hipError_t launch_prefill_fp8(const LoraArgs& p, const uint16_t* tg, int64_t ldt, void* scratch, int terms);

hipError_t launch_decode(const LoraArgs& p);
size_t decode_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, int w_dtype);
bool decode_supported(const LoraArgs& p);
bool decode_groups_supported(const LoraArgs& p);
size_t decode_grouped_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, int groups, int w_dtype);

// Decode-step fusions of the decode kernel (bit 0: RMSNorm prologue on x, bit 1: SwiGLU
// epilogue over interleaved gate/up rows, bit 2: residual-add epilogue).
struct FusedArgs {
  int fuse;
  const void* nw; float eps;      // RMSNorm weight [K] and epsilon
  const void* res; int64_t ldr;   // residual added to the output
};
bool decode_fused_supported(const LoraArgs& p, const FusedArgs& f);
hipError_t launch_decode_fused(const LoraArgs& p, const FusedArgs& f);
// A chain of decode launches in one persistent launch (n stages, each a LoraArgs with its
// FusedArgs; fuse 0 is the plain or grouped form). after_prev[s]: stage s waits for stage
// s - 1. The workspace holds the counter prefix, the stages' flag words and their hand-off
// regions; its sticky failure word is a 32-bit word at decode_chain_err_offset().
bool decode_chain_supported(int64_t M, int n, const LoraArgs* ps, const FusedArgs* fs);
size_t decode_chain_workspace_bytes(int64_t M, int n, const LoraArgs* ps, const FusedArgs* fs);
hipError_t launch_decode_chain(int64_t M, int n, const LoraArgs* ps, const FusedArgs* fs, const int* after_prev,
                               void* ws, hipStream_t stream);
size_t decode_chain_err_offset();
// The tied output head fused with the greedy argmax: out[m] = argmax_n bf16(x[m] . W[n]),
// no logits written. `keys` (decode_argmax_keys_bytes(M) bytes) holds the 64-bit keys of
// the arrival groups and their counters, zero before a launch and after it.
bool decode_argmax_supported(const LoraArgs& p);
size_t decode_argmax_keys_bytes(int64_t M);
hipError_t launch_decode_argmax(const LoraArgs& p, void* keys, int64_t* out);

hipError_t launch_generic(const LoraArgs& p);

hipError_t launch_factorized_embedding(const int64_t* ids, int64_t n_ids, const void* emb,
                                       int64_t lde, int64_t vocab, int64_t k, const void* proj,
                                       int64_t ldp, int64_t hidden, void* out, int64_t ldo,
                                       hipStream_t stream);

// Largest M routed to the decode-shaped (skinny) kernels: every form (fused, fp8 base, the
// greedy head) up to kDecodeMaxM; the plain bf16 wide form (five token blocks, four waves
// along K, x walked in passes) up to kDecodePlainMaxM only when WSL_OPT_DECODE_WIDE asks for
// it: the prefill path's in-launch split-K form is faster from 65 tokens (1.7B layer,
// grouped: 2.24 against 2.46 ms at 65 tokens, 2.25 against 2.61 at 72).
constexpr int64_t kDecodeMaxM = 64;
constexpr int64_t kDecodePlainMaxM = 72;

// Every workspace starts with this many bytes of counters: the decode path's launch counter
// in its first 1 KB, and from kRedCntOff the prefill path's arrival counters of the
// in-launch split-K form (one 32-bit word per tile). They must be zero when the workspace
// is first used; every launch leaves them valid (its counters back at zero) for the next.
// Path-specific scratch follows the prefix.
constexpr size_t kCounterBytes = 65536;
constexpr size_t kRedCntOff = 4096;
constexpr int64_t kRedMaxTiles = (int64_t)((kCounterBytes - kRedCntOff) / 4);

}  // namespace wsl
