// Generic fused-LoRA linear for shapes the MFMA kernels do not take (unaligned
// pointers or leading dimensions, K not a multiple of the K tile). Same arithmetic
// contract as the fast paths: fp32 accumulation, T = bf16(s * x.A^T) rounded once,
// y = bf16((x.W^T) * w_scale + T.B^T).
#include "wsl_common.h"

namespace wsl {
namespace {

constexpr int GT = 16;  // 16x16 output tile per workgroup, K staged through LDS

__device__ __forceinline__ float load_x(const uint16_t* p) { return bf16_bits_to_f32(*p); }

__device__ __forceinline__ float load_w(const void* w, int w_dtype, int64_t idx) {
  if (w_dtype == kBF16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(w)[idx]);
  uint32_t q = reinterpret_cast<const uint8_t*>(w)[idx];
  auto f = __builtin_amdgcn_cvt_pk_f32_fp8((int)q, false);
  return f[0];
}

// T[m][j] = bf16(s * sum_k x[m][k] * A[j][k]); one thread per (m, j).
__global__ void __launch_bounds__(256) generic_down_kernel(const uint16_t* __restrict__ x,
                                                           int64_t ldx,
                                                           const uint16_t* __restrict__ a,
                                                           int64_t lda, float s,
                                                           uint16_t* __restrict__ t, int64_t M,
                                                           int64_t K, int64_t r) {
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * r) return;
  int64_t m = idx / r, j = idx % r;
  const uint16_t* xr = x + m * ldx;
  const uint16_t* ar = a + j * lda;
  float acc = 0.f;
  for (int64_t k = 0; k < K; ++k) acc += load_x(xr + k) * load_x(ar + k);
  t[m * r + j] = f32_to_bf16_bits(s * acc);
}

__global__ void __launch_bounds__(GT* GT) generic_main_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const int64_t* __restrict__ gidx, int64_t grows, const void* __restrict__ w, int64_t ldw,
    int w_dtype, const float* __restrict__ w_scale, const uint16_t* __restrict__ t,
    const uint16_t* __restrict__ b, int64_t ldb, uint16_t* __restrict__ y, int64_t ldy,
    int64_t M, int64_t N, int64_t K, int64_t r, RowMap wmap) {
  __shared__ float xs[GT][GT + 1];
  __shared__ float ws[GT][GT + 1];
  const int tx = threadIdx.x % GT, ty = threadIdx.x / GT;
  const int64_t m0 = (int64_t)blockIdx.y * GT, n0 = (int64_t)blockIdx.x * GT;
  const int64_t m = m0 + ty, n = n0 + tx;
  float acc = 0.f;
  if (w != nullptr) {
    for (int64_t k0 = 0; k0 < K; k0 += GT) {
      // xs[row][kk] = x[m0+row][k0+kk]; ws[col][kk] = W[n0+col][k0+kk]
      int64_t kx = k0 + tx;
      float xv = 0.f;
      if (m0 + ty < M && kx < K) {
        if (gidx != nullptr) {
          const int64_t id = gidx[m0 + ty];
          if (id >= 0 && id < grows) xv = load_x(x + id * ldx + kx);
        } else {
          xv = load_x(x + (m0 + ty) * ldx + kx);
        }
      }
      xs[ty][tx] = xv;
      ws[ty][tx] = (n0 + ty < N && kx < K) ? load_w(w, w_dtype, (int64_t)map_row((int)(n0 + ty), wmap) * ldw + kx) : 0.f;
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < GT; ++kk) acc += xs[ty][kk] * ws[tx][kk];
      __syncthreads();
    }
  }
  if (m >= M || n >= N) return;
  if (w_scale != nullptr) acc *= w_scale[map_row((int)n, wmap)];
  if (r > 0) {
    const uint16_t* tr = t + m * r;
    const uint16_t* br = b + n * ldb;
    for (int64_t j = 0; j < r; ++j) acc += bf16_bits_to_f32(tr[j]) * bf16_bits_to_f32(br[j]);
  }
  y[m * ldy + n] = f32_to_bf16_bits(acc);
}

}  // namespace

size_t generic_workspace_bytes(int64_t M, int64_t r) { return (size_t)(M * r * 2); }

hipError_t launch_generic(const LoraArgs& p) {
  uint16_t* t = reinterpret_cast<uint16_t*>(p.ws);
  if (p.r > 0) {
    int64_t n = p.M * p.r;
    generic_down_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, p.stream>>>(
        reinterpret_cast<const uint16_t*>(p.x), p.ldx, reinterpret_cast<const uint16_t*>(p.a),
        p.lda, p.scale, t, p.M, p.K, p.r);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  dim3 grid((unsigned)((p.N + GT - 1) / GT), (unsigned)((p.M + GT - 1) / GT));
  generic_main_kernel<<<grid, dim3(GT * GT), 0, p.stream>>>(
      reinterpret_cast<const uint16_t*>(p.x), p.ldx, p.gather, p.gather_rows, p.w, p.ldw,
      p.w_dtype, p.w_scale, t,
      reinterpret_cast<const uint16_t*>(p.b), p.ldb, reinterpret_cast<uint16_t*>(p.y), p.ldy,
      p.M, p.N, p.K, p.r, p.wmap);
  return hipGetLastError();
}

}  // namespace wsl
