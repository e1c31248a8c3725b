// Weight gradients of the fused LoRA linear (y = x . W^T + s (x . A^T) . B^T) on gfx950:
//
//   dW = gy^T . x            [N, K]
//   dA = s (gy . B)^T . x    [r, K]
//   dB = s gy^T . (x . A^T)  [N, r]
//
// dW reduces over the M tokens of two operands that store tokens as rows. The fused kernel's
// tile loop takes them in that form (TN: the tiles go into LDS as they lie and each MFMA
// fragment is read with gfx950's transposing LDS reads), so neither operand is copied. An
// output too small to fill the 256 CUs splits the token reduction into equal parts (fp32
// partials) that a reduce kernel sums in split order (deterministic), rounding once to bf16.
//
// With dW at hand, dA and dB follow from it by associativity, as products over K or N
// instead of over the tokens:
//
//   dB = s (gy^T . x) . A^T = s dW . A^T        dA = s B^T . (gy^T . x) = s B^T . dW
//
// 2 N K r multiply-adds each instead of 2 M r (N + K) for the rank projections T = x . A^T,
// U = gy . B and their products: both read the bf16 dW (dA through its transpose) and
// nothing of size M. Without dW (a frozen base) they take the token route instead:
// T = bf16(s x . A^T) and U = bf16(s gy . B) from the forward's rank pre-pass, then
// dB = gy^T . T and dA = U^T . x as token-major products.
//
// The reference has no backward of its own: torch autograd differentiates LoRAModule.forward
// (torchtitan/models/llama3/model/model.py:189-192) and the base nn.Linear (:257-273)
// composed by broadcast_add (:392-398); the trainer runs it at torchtitan/train.py:456.
#include <algorithm>

#include "wsl_common.h"

namespace wsl {

namespace {

constexpr int TT = 64;       // transpose tile: 64 rows x 64 columns
constexpr int TS = TT + 2;   // its LDS row stride in bf16 (odd word count: spread banks)

// dst[c][i] = src[i][c] for i < R and 0 for R <= i < Rp, c < C (B^T and dW^T here, Rp = R).
// 16-byte global accesses both ways (C % 8 == 0, Rp % 8 == 0, 16-byte aligned rows).
struct TransposeJob {
  const uint16_t* src;
  int64_t lds_, R, C;
  uint16_t* dst;
  int64_t ldd, Rp;
};

// The 64 x 64 tile (bx, by) of one job, staged through `tile`.
__device__ __forceinline__ void transpose_tile(const TransposeJob& j, int64_t bx, int64_t by, uint32_t* tile) {
  const uint16_t* __restrict__ src = j.src;
  uint16_t* __restrict__ dst = j.dst;
  const int64_t lds_ = j.lds_, R = j.R, C = j.C, ldd = j.ldd, Rp = j.Rp;
  const uint16_t* t16 = reinterpret_cast<const uint16_t*>(tile);
  const int64_t r0 = by * TT, c0 = bx * TT;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = tid + 256 * i, row = idx >> 3, ch = idx & 7;
    const int64_t r = r0 + row, c = c0 + ch * 8;
    u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
    if (r < R && c < C) v = *reinterpret_cast<const u32x4_t*>(src + r * lds_ + c);
    uint32_t* d = tile + (row * TS + ch * 8) / 2;  // TS even, ch * 8 even: word aligned
    d[0] = v[0]; d[1] = v[1]; d[2] = v[2]; d[3] = v[3];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = tid + 256 * i, q = idx & 7, c = idx >> 3;  // 8 lanes: one 128-byte output row piece
    if (c0 + c >= C || r0 + q * 8 >= Rp) continue;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = (uint32_t)t16[(q * 8 + 2 * j) * TS + c] | ((uint32_t)t16[(q * 8 + 2 * j + 1) * TS + c] << 16);
    *reinterpret_cast<u32x4_t*>(dst + (c0 + c) * ldd + r0 + q * 8) = u32x4_t{w[0], w[1], w[2], w[3]};
  }
}

__global__ void __launch_bounds__(256) transpose_pad_kernel(const TransposeJob j) {
  __shared__ uint32_t tile[TT * TS / 2];
  transpose_tile(j, blockIdx.x, blockIdx.y, tile);
}

// Two jobs in one launch (blockIdx.z picks the job; tiles past a job's extent exit).
__global__ void __launch_bounds__(256) transpose_pair_kernel(const TransposeJob j0, const TransposeJob j1) {
  __shared__ uint32_t tile[TT * TS / 2];
  const TransposeJob& j = blockIdx.z == 0 ? j0 : j1;
  if ((int64_t)blockIdx.x * TT >= j.C || (int64_t)blockIdx.y * TT >= j.Rp) return;
  transpose_tile(j, blockIdx.x, blockIdx.y, tile);
}

// Four bf16 of row-major `d` (8-byte pieces when `vec`).
__device__ __forceinline__ void store4(uint16_t* d, f32x4_t v, bool vec) {
  if (vec) {
    *reinterpret_cast<uint2*>(d) = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  } else {
    d[0] = f32_to_bf16_bits(v[0]); d[1] = f32_to_bf16_bits(v[1]);
    d[2] = f32_to_bf16_bits(v[2]); d[3] = f32_to_bf16_bits(v[3]);
  }
}

// sum over q of p[q * slice .. + 4) in split order, four loads in flight at a time (16-byte
// aligned p, slice % 4 == 0).
__device__ __forceinline__ f32x4_t sum_splits(const float* p, int64_t slice, int splits) {
  const f32x4_t* pv = reinterpret_cast<const f32x4_t*>(p);
  const int64_t sv = slice / 4;
  f32x4_t a = pv[0];
  int q = 1;
  for (; q + 4 <= splits; q += 4) {
    const f32x4_t a0 = pv[q * sv], a1 = pv[(q + 1) * sv], a2 = pv[(q + 2) * sv], a3 = pv[(q + 3) * sv];
    a += a0; a += a1; a += a2; a += a3;
  }
  for (; q < splits; ++q) a += pv[q * sv];
  return a;
}

// dst = bf16(scale * sum over the splits of part[s]) for an fp32 [splits][rows][cols] partial
// product, splits in order; four consecutive columns per thread (cols % 4 == 0).
__global__ void __launch_bounds__(256) split_sum_kernel(const float* __restrict__ part, int splits, int64_t rows,
                                                       int64_t cols, float scale, uint16_t* __restrict__ dst,
                                                       int64_t ldd, int vec) {
  const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  const int64_t slice = rows * cols;
  if (e >= slice) return;
  store4(dst + (e / cols) * ldd + e % cols, sum_splits(part + e, slice, splits) * scale, vec != 0);
}

// dW = bf16(sum over the splits of part[s]) ([splits][N][K] fp32, splits in order) to the
// caller's dw (row stride lddw, 8-byte pieces when `vec`), to the contiguous copy dwc
// [N][K] when given, and transposed to dwt [K][N] when given. 64 x 64 tiles (N % 64 ==
// K % 64 == 0); the transpose goes through LDS as in transpose_pad_kernel.
__global__ void __launch_bounds__(256) dw_reduce_kernel(const float* __restrict__ part, int splits, int64_t N,
                                                       int64_t K, uint16_t* __restrict__ dw, int64_t lddw, int vec,
                                                       uint16_t* __restrict__ dwc, uint16_t* __restrict__ dwt) {
  __shared__ uint32_t tile[TT * TS / 2];
  const uint16_t* t16 = reinterpret_cast<const uint16_t*>(tile);
  const int64_t n0 = (int64_t)blockIdx.y * TT, k0 = (int64_t)blockIdx.x * TT;
  const int tid = threadIdx.x;
  const int64_t slice = N * K;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = tid / 16 + 16 * i, col = (tid % 16) * 4;
    const int64_t e = (n0 + row) * K + k0 + col;
    const f32x4_t v = sum_splits(part + e, slice, splits);
    store4(dw + (n0 + row) * lddw + k0 + col, v, vec != 0);
    const uint32_t lo = pack_bf16x2(v[0], v[1]), hi = pack_bf16x2(v[2], v[3]);
    if (dwc != nullptr) *reinterpret_cast<uint2*>(dwc + e) = uint2{lo, hi};
    uint32_t* d = tile + (row * TS + col) / 2;
    d[0] = lo; d[1] = hi;
  }
  if (dwt == nullptr) return;  // uniform over the workgroup
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = tid + 256 * i, q = idx & 7, c = idx >> 3;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = (uint32_t)t16[(q * 8 + 2 * j) * TS + c] | ((uint32_t)t16[(q * 8 + 2 * j + 1) * TS + c] << 16);
    *reinterpret_cast<u32x4_t*>(dwt + (k0 + c) * N + n0 + q * 8) = u32x4_t{w[0], w[1], w[2], w[3]};
  }
}

hipError_t transpose_pad(const void* src, int64_t lds_, int64_t R, int64_t C, uint16_t* dst, int64_t ldd,
                         int64_t Rp, hipStream_t st) {
  if (C == 0 || Rp == 0) return hipSuccess;
  const dim3 grid((unsigned)((C + TT - 1) / TT), (unsigned)((Rp + TT - 1) / TT));
  transpose_pad_kernel<<<grid, dim3(256), 0, st>>>(TransposeJob{reinterpret_cast<const uint16_t*>(src), lds_, R, C,
                                                                dst, ldd, Rp});
  return hipGetLastError();
}

// Both transposes of the input gradient's rank factors in one launch.
hipError_t transpose_pair(const TransposeJob& j0, const TransposeJob& j1, hipStream_t st) {
  const int64_t gx = std::max((j0.C + TT - 1) / TT, (j1.C + TT - 1) / TT);
  const int64_t gy = std::max((j0.Rp + TT - 1) / TT, (j1.Rp + TT - 1) / TT);
  transpose_pair_kernel<<<dim3((unsigned)gx, (unsigned)gy, 2), dim3(256), 0, st>>>(j0, j1);
  return hipGetLastError();
}

// ---- Layouts the tile kernels do not take (K or N off the 64 grid, r not a multiple of 8,
// unaligned rows): the token route on scalar kernels, same contract ----

// t[m][j] = bf16(s * sum_k x[m][k] * f[j * fj + k * fk]) for m < M, j < r: T = x . A^T
// (fj = lda, fk = 1) or U = gy . B (fj = 1, fk = ldb). One thread per (m, j), k in order.
__global__ void __launch_bounds__(256) generic_rank_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                          const uint16_t* __restrict__ f, int64_t fj, int64_t fk,
                                                          float s, uint16_t* __restrict__ t, int64_t M, int64_t K,
                                                          int64_t r) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= M * r) return;
  const int64_t m = idx / r, j = idx % r;
  const uint16_t* xr = x + m * ldx;
  const uint16_t* fr = f + j * fj;
  float acc = 0.f;
  for (int64_t k = 0; k < K; ++k) acc += bf16_bits_to_f32(xr[k]) * bf16_bits_to_f32(fr[k * fk]);
  t[m * r + j] = f32_to_bf16_bits(s * acc);
}

// c[i][j] = bf16(sum_m p[m][i] * q[m][j]) over the M token rows of two token-major operands
// (dW = gy^T . x, dA = U^T . x, dB = gy^T . T). A workgroup owns a 64 x 64 output tile, each
// thread 4 x 4 outputs; 16 tokens at a time are staged through LDS. Every output is summed
// by one thread in token order, so the result is deterministic.
constexpr int GW = 64, GWK = 16;
__global__ void __launch_bounds__(256) generic_token_product_kernel(const uint16_t* __restrict__ p, int64_t ldp,
                                                                   const uint16_t* __restrict__ q, int64_t ldq,
                                                                   int64_t M, int64_t I, int64_t J,
                                                                   uint16_t* __restrict__ c, int64_t ldc) {
  __shared__ float ps[GWK][GW + 1];
  __shared__ float qs[GWK][GW + 1];
  const int tid = threadIdx.x;
  const int ti = tid / 16, tj = tid % 16;  // this thread's outputs: rows ti + 16 u, columns tj + 16 v
  const int64_t i0 = (int64_t)blockIdx.y * GW, j0 = (int64_t)blockIdx.x * GW;
  float acc[4][4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[u][v] = 0.f;
  for (int64_t m0 = 0; m0 < M; m0 += GWK) {
    // 16 tokens x 64 columns of each operand: four elements per thread, columns fastest
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = tid + 256 * e, row = idx / GW, col = idx % GW;
      const int64_t m = m0 + row;
      ps[row][col] = (m < M && i0 + col < I) ? bf16_bits_to_f32(p[m * ldp + i0 + col]) : 0.f;
      qs[row][col] = (m < M && j0 + col < J) ? bf16_bits_to_f32(q[m * ldq + j0 + col]) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < GWK; ++kk) {
      float pv[4], qv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) pv[u] = ps[kk][ti + 16 * u];
#pragma unroll
      for (int v = 0; v < 4; ++v) qv[v] = qs[kk][tj + 16 * v];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[u][v] += pv[u] * qv[v];
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t i = i0 + ti + 16 * u;
    if (i >= I) continue;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t j = j0 + tj + 16 * v;
      if (j < J) c[i * ldc + j] = f32_to_bf16_bits(acc[u][v]);
    }
  }
}

size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }
bool al16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

// Workspace plan. It depends on the sizes only, so the workspace query needs no flags: the
// union of both routes' buffers.
struct Plan {
  int sw;          // token splits of the dW product
  int sb, sa;      // token route: token splits of the dB and dA products
  int sdb, sda;    // dW route: splits of dB = s dW . A^T (over K) and dA = s B^T . dW (over N)
  size_t off_t, off_u, off_bt, off_dwc, off_dwt, off_part, total;
};

Plan make_plan(int64_t M, int64_t N, int64_t K, int64_t r) {
  Plan L{};
  const int64_t nk = (M + 63) / 64;
  L.sw = product_splits(N, K, nk, false);
  L.sb = r > 0 ? product_splits(N, r, nk, false) : 1;
  L.sa = r > 0 ? product_splits(r, K, nk, false) : 1;
  L.sdb = r > 0 ? product_splits(N, r, K / 64, true) : 1;
  L.sda = r > 0 ? product_splits(r, K, N / 64, true) : 1;
  size_t off = 0;
  L.off_t = off;   off = a256(off + (r > 0 ? rank_prepass_bytes(M, K, r) : 0));
  L.off_u = off;   off = a256(off + (r > 0 ? rank_prepass_bytes(M, N, r) : 0));
  L.off_bt = off;  off = a256(off + (size_t)r * N * 2);
  L.off_dwc = off; off = a256(off + (r > 0 ? (size_t)N * K * 2 : 0));
  L.off_dwt = off; off = a256(off + (r > 0 ? (size_t)N * K * 2 : 0));
  L.off_part = off;
  size_t part = (size_t)L.sw * N * K;  // worst case: any product may go through partials
  const size_t cand[4] = {(size_t)L.sb * N * r, (size_t)L.sa * r * K, (size_t)L.sdb * N * r, (size_t)L.sda * r * K};
  for (size_t c : cand) part = c > part ? c : part;
  L.total = a256(off + part * 4);
  return L;
}

}  // namespace

// Shapes and layouts the tile kernels of the weight-gradient path take: K and N on the
// 64-element tile grid (the reductions of the dA and dB products and of the token route's
// pre-passes), ranks in multiples of 8, 16-byte aligned rows, and sizes within the tile
// kernel's int range. Every other layout takes the generic route above.
bool weight_grads_supported(const LoraArgs& p, const void* gy, int64_t ldg) {
  if (p.M < 1 || p.K % 64 != 0 || p.N % 64 != 0 || p.r % 8 != 0) return false;
  if (p.M > ((int64_t)1 << 22) - 2048 || p.N > ((int64_t)1 << 22) || p.K > ((int64_t)1 << 22)) return false;
  if (!al16(p.x) || p.ldx % 8 != 0 || !al16(gy) || ldg % 8 != 0) return false;
  if (p.ldx > ((int64_t)1 << 22) || ldg > ((int64_t)1 << 22)) return false;
  if (p.r > 0 && (!al16(p.a) || p.lda % 8 != 0 || !al16(p.b) || p.ldb % 8 != 0 || p.lda > ((int64_t)1 << 22)))
    return false;
  return true;
}

size_t weight_grads_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, bool need_w, bool need_ab) {
  (void)need_w;
  return make_plan(M, N, K, need_ab ? r : 0).total;
}

namespace {
// The generic route: T = bf16(s x . A^T) and U = bf16(s gy . B) into the workspace's T and U
// regions, then dW = gy^T . x, dB = gy^T . T and dA = U^T . x over the tokens.
hipError_t launch_weight_grads_generic(const LoraArgs& p, const void* gy, int64_t ldg, void* dw, int64_t lddw,
                                       void* da, int64_t ldda, void* db, int64_t lddb, int64_t r, const Plan& L) {
  const int64_t M = p.M, N = p.N, K = p.K;
  char* ws = reinterpret_cast<char*>(p.ws);
  uint16_t* T = reinterpret_cast<uint16_t*>(ws + L.off_t);
  uint16_t* U = reinterpret_cast<uint16_t*>(ws + L.off_u);
  const uint16_t* x = reinterpret_cast<const uint16_t*>(p.x);
  const uint16_t* g = reinterpret_cast<const uint16_t*>(gy);
  const hipStream_t st = p.stream;
  const dim3 rank_grid((unsigned)((M * r + 255) / 256));
  auto product = [&](const uint16_t* pp, int64_t ldp, int64_t I, const uint16_t* qq, int64_t ldq, int64_t J,
                     void* dst, int64_t ldd) {
    const dim3 grid((unsigned)((J + GW - 1) / GW), (unsigned)((I + GW - 1) / GW));
    generic_token_product_kernel<<<grid, dim3(256), 0, st>>>(pp, ldp, qq, ldq, M, I, J, reinterpret_cast<uint16_t*>(dst),
                                                             ldd);
    return hipGetLastError();
  };
  hipError_t e = hipSuccess;
  if (dw != nullptr) e = product(g, ldg, N, x, p.ldx, K, dw, lddw);
  if (e == hipSuccess && db != nullptr) {
    generic_rank_kernel<<<rank_grid, dim3(256), 0, st>>>(x, p.ldx, reinterpret_cast<const uint16_t*>(p.a), p.lda, 1,
                                                         p.scale, T, M, K, r);
    e = hipGetLastError();
    if (e == hipSuccess) e = product(g, ldg, N, T, r, r, db, lddb);
  }
  if (e == hipSuccess && da != nullptr) {
    generic_rank_kernel<<<rank_grid, dim3(256), 0, st>>>(g, ldg, reinterpret_cast<const uint16_t*>(p.b), 1, p.ldb,
                                                         p.scale, U, M, N, r);
    e = hipGetLastError();
    if (e == hipSuccess) e = product(U, r, r, x, p.ldx, K, da, ldda);
  }
  return e;
}
}  // namespace

// ---- Input gradient: dX = dY . W + s (dY . B) . A, W read where it lies ----
// The forward-shaped problem of dX (x' = dY, reduction K' = N, N' = K output columns) runs
// on the prefill kernel's WT form: W's rows are the reduction, so its tiles go into LDS as
// they lie and its fragments are transposing reads; no copy of W. The rank factors take the
// places of the forward's: A' = B^T [r, N] and B' = A^T [K, r], transposed into the
// workspace after the prefill scratch (r (N + K) bf16).
namespace {
LoraArgs wt_problem(const LoraArgs& p) {
  LoraArgs q = p;
  q.K = p.N;
  q.N = p.K;
  return q;
}
size_t a256b(size_t v) { return (v + 255) & ~(size_t)255; }
}  // namespace

bool bwd_input_supported(const LoraArgs& p) {
  if (p.r > 0 && (p.N % 8 != 0 || p.K % 8 != 0 || !al16(p.a) || p.lda % 8 != 0 || !al16(p.b) || p.ldb % 8 != 0))
    return false;
  LoraArgs q = wt_problem(p);
  // the transposed factors stand in for a and b (aligned, tight leading dimensions)
  static char kAligned[16] __attribute__((aligned(16))) = {0};
  q.a = p.r > 0 ? kAligned : nullptr;
  q.lda = p.N;
  q.b = p.r > 0 ? kAligned : nullptr;
  q.ldb = p.r;
  return prefill_wt_supported(q);
}

size_t bwd_input_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r) {
  return a256b(prefill_workspace_bytes(M, K, N, r, kBF16)) + a256b((size_t)r * N * 2) + (size_t)K * r * 2;
}

hipError_t launch_bwd_input(const LoraArgs& p) {
  LoraArgs q = wt_problem(p);
  hipError_t e = hipSuccess;
  if (p.r > 0) {
    char* base = reinterpret_cast<char*>(p.ws) + a256b(prefill_workspace_bytes(p.M, p.K, p.N, p.r, kBF16));
    uint16_t* bt = reinterpret_cast<uint16_t*>(base);
    uint16_t* at = reinterpret_cast<uint16_t*>(base + a256b((size_t)p.r * p.N * 2));
    // B [N, r] -> B^T [r, N] and A [r, K] -> A^T [K, r], one launch
    e = transpose_pair(TransposeJob{reinterpret_cast<const uint16_t*>(p.b), p.ldb, p.N, p.r, bt, p.N, p.N},
                       TransposeJob{reinterpret_cast<const uint16_t*>(p.a), p.lda, p.r, p.K, at, p.r, p.r}, p.stream);
    q.a = bt;
    q.lda = p.N;
    q.b = at;
    q.ldb = p.r;
  }
  if (e == hipSuccess) e = launch_prefill_wt(q);
  return e;
}

hipError_t launch_weight_grads(const LoraArgs& p, const void* gy, int64_t ldg, void* dw, int64_t lddw, void* da,
                               int64_t ldda, void* db, int64_t lddb) {
  const int64_t M = p.M, N = p.N, K = p.K;
  const int64_t r = (da != nullptr || db != nullptr) ? p.r : 0;
  if (r == 0) da = db = nullptr;
  if (dw == nullptr && r == 0) return hipSuccess;
  const Plan L = make_plan(M, N, K, r);
  if (!weight_grads_supported(p, gy, ldg)) return launch_weight_grads_generic(p, gy, ldg, dw, lddw, da, ldda, db, lddb, r, L);
  char* ws = reinterpret_cast<char*>(p.ws);
  uint16_t* T = reinterpret_cast<uint16_t*>(ws + L.off_t);
  uint16_t* U = reinterpret_cast<uint16_t*>(ws + L.off_u);
  uint16_t* Bt = reinterpret_cast<uint16_t*>(ws + L.off_bt);
  uint16_t* dwc = reinterpret_cast<uint16_t*>(ws + L.off_dwc);
  uint16_t* dwt = reinterpret_cast<uint16_t*>(ws + L.off_dwt);
  float* part = reinterpret_cast<float*>(ws + L.off_part);
  const hipStream_t st = p.stream;
  const int64_t nkt = (M + 63) / 64;  // 64-token K tiles
  hipError_t e = hipSuccess;

  auto vec_ok = [](const void* dst, int64_t ldd) { return (reinterpret_cast<uintptr_t>(dst) & 7u) == 0 && ldd % 4 == 0; };
  // dst = bf16(scale * sum_s part[s]) [rows, cols] from the partial products
  auto reduce = [&](int splits, int64_t rows, int64_t cols, float scale, void* dst, int64_t ldd, bool vec) {
    const int64_t n4 = rows * cols / 4;
    split_sum_kernel<<<dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st>>>(
        part, splits, rows, cols, scale, reinterpret_cast<uint16_t*>(dst), ldd, vec ? 1 : 0);
    return hipGetLastError();
  };
  // y' = scale * x' . W'^T, x' and W' rows `red` long: straight to bf16 when unsplit and the
  // destination takes the tile store's 8-byte pieces, else through fp32 partials
  auto product = [&](const void* xa, int64_t ldxa, int64_t rows, const void* wb, int64_t ldwb, int64_t cols,
                     int64_t red, int splits, float scale, void* dst, int64_t ldd) -> hipError_t {
    LoraArgs q = p;
    q.x = xa; q.ldx = ldxa; q.w = wb; q.ldw = ldwb; q.M = rows; q.N = cols; q.yscale = scale;
    const bool vec = vec_ok(dst, ldd);
    if (splits == 1 && vec) {
      q.K = red; q.y = dst; q.ldy = ldd;
      return launch_product(q, nullptr, 1);
    }
    q.K = red / splits;
    const hipError_t err = launch_product(q, part, splits);
    return err != hipSuccess ? err : reduce(splits, rows, cols, scale, dst, ldd, vec);
  };
  // Token splits as launched: equal whole 64-token tiles, none starting past the tokens.
  auto tn_splits = [&](int splits, int64_t* per) {
    const int64_t kt = (nkt + splits - 1) / splits;
    *per = kt * 64;
    return (int)((nkt + kt - 1) / kt);
  };
  // the same over the tokens with token-major operands: x'[m][t] = xa[t * ldxa + m],
  // W'[n][t] = wb[t * ldwb + n]
  auto product_tn = [&](const void* xa, int64_t ldxa, int64_t rows, const void* wb, int64_t ldwb, int64_t cols,
                        int splits, float scale, void* dst, int64_t ldd) -> hipError_t {
    LoraArgs q = p;
    q.x = xa; q.ldx = ldxa; q.w = wb; q.ldw = ldwb; q.M = rows; q.N = cols; q.yscale = scale;
    const int s = tn_splits(splits, &q.K);
    const bool vec = vec_ok(dst, ldd);
    if (s == 1 && vec) {
      q.y = dst; q.ldy = ldd;
      return launch_product_tn(q, M, nullptr, 1);
    }
    const hipError_t err = launch_product_tn(q, M, part, s);
    return err != hipSuccess ? err : reduce(s, rows, cols, scale, dst, ldd, vec);
  };

  if (dw != nullptr) {
    // ---- dW route: dW over the tokens, then dB = s dW . A^T and dA = s B^T . dW ----
    int64_t per = 0;
    const int sw = tn_splits(L.sw, &per);
    const bool direct = sw == 1 && al16(dw) && lddw % 8 == 0;
    const uint16_t* dws = reinterpret_cast<const uint16_t*>(dw);  // bf16 dW rows for dB
    int64_t ldws = lddw;
    if (direct) {
      e = product_tn(gy, ldg, N, p.x, p.ldx, K, 1, 1.f, dw, lddw);
      if (e == hipSuccess && da != nullptr) e = transpose_pad(dw, lddw, N, K, dwt, N, N, st);
    } else {
      LoraArgs q = p;
      q.x = gy; q.ldx = ldg; q.w = p.x; q.ldw = p.ldx; q.M = N; q.N = K; q.K = per;
      e = launch_product_tn(q, M, part, sw);
      if (e == hipSuccess) {
        dw_reduce_kernel<<<dim3((unsigned)(K / TT), (unsigned)(N / TT)), dim3(256), 0, st>>>(
            part, sw, N, K, reinterpret_cast<uint16_t*>(dw), lddw, vec_ok(dw, lddw) ? 1 : 0,
            db != nullptr ? dwc : nullptr, da != nullptr ? dwt : nullptr);
        e = hipGetLastError();
      }
      dws = dwc;
      ldws = K;
    }
    if (e == hipSuccess && db != nullptr) e = product(dws, ldws, N, p.a, p.lda, r, K, L.sdb, p.scale, db, lddb);
    if (e == hipSuccess && da != nullptr) {
      e = transpose_pad(p.b, p.ldb, N, r, Bt, N, N, st);
      if (e == hipSuccess) e = product(Bt, N, r, dwt, N, K, N, L.sda, p.scale, da, ldda);
    }
    return e;
  }

  // ---- token route (no dW): T, U by the rank pre-pass, token-major products ----
  if (db != nullptr) {  // dB = gy^T . T, T = bf16(s x . A^T)
    LoraArgs q = p;
    q.groups = 1;
    e = rank_prepass(q, T);
    if (e == hipSuccess) e = product_tn(gy, ldg, N, T, r, r, L.sb, 1.f, db, lddb);
    if (e != hipSuccess) return e;
  }
  if (da != nullptr) {  // dA = U^T . x, U = bf16(s gy . B) with B^T [r, N] in the place of A
    e = transpose_pad(p.b, p.ldb, N, r, Bt, N, N, st);
    if (e != hipSuccess) return e;
    LoraArgs q = p;
    q.x = gy; q.ldx = ldg; q.K = N; q.a = Bt; q.lda = N; q.groups = 1;
    e = rank_prepass(q, U);
    if (e == hipSuccess) e = product_tn(U, r, r, p.x, p.ldx, K, L.sa, 1.f, da, ldda);
  }
  return e;
}

}  // namespace wsl
