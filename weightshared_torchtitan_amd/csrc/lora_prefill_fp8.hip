// Prefill-shaped fused LoRA linear with an fp8 (OCP e4m3fn) base weight on gfx950's fp8
// matrix cores:
//
//   y[M,N] = 2^e[m] * (sum_t 2^(-4 t) xq[t] . Wq^T) * diag(w_scale) + T . B^T,
//   T = bf16(s * x . A^T)
//
// The activations are split per token by fp8_split_kernel: e[m] is the smallest power of
// two that brings max|x[m]| under 448, xq[0] = e4m3(x 2^-e) and, with two terms,
// xq[1] = e4m3((x 2^-e - xq[0]) 2^4), the rounding residual one e4m3 step down. Two terms
// carry a bf16 activation to within 2^-8 of itself, so the result keeps the weight-only fp8
// error; one term (an opt-in) halves the MFMA work and adds e4m3 rounding of x.
//
// Main loop. v_mfma_scale_f32_32x32x64_f8f6f4 multiplies 32 x 64 fp8 tiles of W (the "A"
// operand, rows n) and of x (the "B" operand, rows m) into a 32 x 32 fp32 block; its E8M0
// scale operand of the x tiles carries the 2^-4 of the residual term (2^0 for the first),
// so both terms accumulate into the same registers. Lane l of a fragment holds row l % 32,
// bytes 0-15 = k [16h, 16h + 16) and bytes 16-31 = k [32 + 16h, 48 + 16h) for h = l / 32:
// the lane pair (l, l + 32) then covers the 32-wide k block the hardware applies one scale
// to. A workgroup of 8 waves owns a 256 x 256 output tile (128(n) x 64(m) per wave, as the
// bf16 kernel's largest tile). K is walked 64 at a time (one MFMA k step) through three LDS
// stages filled by global_load_lds_dwordx4 (64-byte rows, XOR swizzle on row bits 2-3), two
// K tiles in flight while one is multiplied.
//
// Epilogue: the fp32 block sums are scaled by 2^e[m] * w_scale[n], the LoRA up-projection
// T . B^T (T from the rank pre-pass of the bf16 path, in the workspace) accumulates on the
// bf16 matrix cores into the same registers, and the tile is staged through LDS and written
// as whole rows, as in the bf16 kernel.
//
// Reference arithmetic being fused: torchtitan/models/llama3/model/model.py:189-192
// (LoRAModule.forward), :392-398 (base projection + broadcast_add, g = 1); the fp8 base is
// this build's weight-only e4m3 scheme (the reference's fp8 is torchao's training recipe,
// torchtitan/components/quantization/float8.py:26-218).
#include <climits>
#include <type_traits>

#include "wsl_common.h"

namespace wsl {
namespace {

typedef __attribute__((address_space(3))) void lds_void_t;
typedef int i32x8_t __attribute__((ext_vector_type(8)));

constexpr int F8_BM = 256, F8_BN = 256;      // output tile
constexpr int F8_NT = 512;                   // 8 waves
constexpr int F8_WNW = 2;                    // waves along n (4 along m)
constexpr int F8_TN = 128, F8_TM = 64;       // wave tile
constexpr int F8_NI = F8_TN / 32, F8_MJ = F8_TM / 32;
constexpr int F8_BK = 64;                    // k (bytes) per K tile: one MFMA k step
constexpr int F8_TILE = F8_BM * F8_BK;       // bytes of one operand tile (x or W): 16 KB
constexpr int F8_S = 3;                      // LDS stages
constexpr int F8_N_XCD = 8;
constexpr int F8_GROUP_M = 4;
constexpr int kLoShift = 4;                  // the residual term carries x's residual * 2^4
constexpr int kE8M0One = 127;                // E8M0 encoding of 2^0

// Byte offset of 16-byte chunk c (0..3) of 64-byte LDS row `row`. A ds_read_b128 is served
// 16 lanes (256 bytes, all 64 banks) at a time; 16 consecutive rows at one chunk index land
// on 16 distinct 16-byte bank groups (4 rows per bank-group cycle, the XOR spreads the 4).
__device__ __forceinline__ int f8_off(int row, int c) { return row * 64 + ((c ^ ((row >> 2) & 3)) << 4); }

// Chunk a lane fetches in a direct fill: lane i lands at LDS slot i % 4 of row 16 g + i / 4.
__device__ __forceinline__ int f8_fill_chunk(int lane) { return (lane & 3) ^ ((lane >> 4) & 3); }

// bf16 LoRA phase: 128-byte rows (64 bf16), XOR swizzle with row bits 1..3 (as the bf16 kernel).
__device__ __forceinline__ int b16_off(int row, int c) { return row * 128 + ((c ^ ((row >> 1) & 7)) << 4); }

__device__ __forceinline__ uint32_t f8_opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

template <int N>
__device__ __forceinline__ void f8_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}

__device__ __forceinline__ void f8_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS reads are complete
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// One fragment: row `row` of an fp8 tile, the lane's two 16-byte k pieces.
__device__ __forceinline__ i32x8_t f8_frag(const char* tile, int row, int h) {
  const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(tile + f8_off(row, h));
  const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(tile + f8_off(row, 2 + h));
  return i32x8_t{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// ---------------------------------------------------------------------------- split
// One workgroup per token row: the row's largest magnitude, its power-of-two exponent e
// (smallest e with max|x| 2^-e <= 448 = 1.75 * 2^8, clamped to [-126, 127]), then the
// codes of every element. All arithmetic is exact but the e4m3 roundings (nearest even).
// The row is read once: each thread keeps its CH chunks of 8 elements in registers across
// the reduction (rows of up to SPLIT_T * 8 * CH elements).
constexpr int SPLIT_T = 256;

__device__ __forceinline__ float split_exponent_scale(float a, int* e_out) {
  int e = 0;
  if (a > 0.f) {
    int ex;
    const float mant = frexpf(a, &ex);  // a = mant * 2^ex, mant in [0.5, 1)
    e = (ex - 1) - 8 + (2.f * mant > 1.75f ? 1 : 0);
    e = e < -126 ? -126 : (e > 127 ? 127 : e);
  }
  *e_out = e;
  return ldexpf(1.f, e);
}

// 8 elements x (already scaled by 2^-e) -> 8 codes of the first term and, with TERMS == 2,
// of the residual term.
template <int TERMS>
__device__ __forceinline__ void split8(const float (&f)[8], uint2& hi, uint2& lo) {
  uint32_t hw[2];
#pragma unroll
  for (int w2 = 0; w2 < 2; ++w2) {
    uint32_t wd = __builtin_amdgcn_cvt_pk_fp8_f32(f[4 * w2], f[4 * w2 + 1], 0, false);
    wd = __builtin_amdgcn_cvt_pk_fp8_f32(f[4 * w2 + 2], f[4 * w2 + 3], wd, true);
    hw[w2] = wd;
  }
  hi = uint2{hw[0], hw[1]};
  if constexpr (TERMS == 2) {
    float r[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t code = (hw[e >> 2] >> ((e & 3) * 8)) & 0xffu;
      r[e] = (f[e] - __builtin_amdgcn_cvt_pk_f32_fp8((int)code, false)[0]) * (float)(1 << kLoShift);
    }
    uint32_t lw[2];
#pragma unroll
    for (int w2 = 0; w2 < 2; ++w2) {
      uint32_t wd = __builtin_amdgcn_cvt_pk_fp8_f32(r[4 * w2], r[4 * w2 + 1], 0, false);
      wd = __builtin_amdgcn_cvt_pk_fp8_f32(r[4 * w2 + 2], r[4 * w2 + 3], wd, true);
      lw[w2] = wd;
    }
    lo = uint2{lw[0], lw[1]};
  }
}

template <int TERMS, int CH>
__global__ void __launch_bounds__(SPLIT_T) fp8_split_kernel(const uint16_t* __restrict__ x, int64_t ldx, int K,
                                                           uint8_t* __restrict__ xq, int64_t term_stride,
                                                           float* __restrict__ sx) {
  __shared__ float red[SPLIT_T / 64];
  const int m = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* xr = x + (int64_t)m * ldx;
  const int nch = K / 8;
  u32x4_t v[CH];
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int c = u * SPLIT_T + tid;
    v[u] = c < nch ? ld_global_16(xr + c * 8) : zero_u32x4();
  }
  float amax = 0.f;
#pragma unroll
  for (int u = 0; u < CH; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(bf16_bits_to_f32((v[u][e >> 1] >> ((e & 1) * 16)) & 0xffffu)));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  float a = red[0];
#pragma unroll
  for (int q = 1; q < SPLIT_T / 64; ++q) a = fmaxf(a, red[q]);
  int e;
  const float s = split_exponent_scale(a, &e);
  if (tid == 0) sx[m] = s;
  const float inv = ldexpf(1.f, -e);  // exact power of two
  uint8_t* q0 = xq + (int64_t)m * K;
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    const int c = u * SPLIT_T + tid;
    if (c >= nch) continue;
    float f[8];
#pragma unroll
    for (int el = 0; el < 8; ++el) f[el] = bf16_bits_to_f32((v[u][el >> 1] >> ((el & 1) * 16)) & 0xffffu) * inv;
    uint2 hi, lo;
    split8<TERMS>(f, hi, lo);
    *reinterpret_cast<uint2*>(q0 + c * 8) = hi;
    if constexpr (TERMS == 2) *reinterpret_cast<uint2*>(q0 + term_stride + c * 8) = lo;
  }
}

// Rows longer than the register-resident form holds: two passes over the row.
template <int TERMS>
__global__ void __launch_bounds__(SPLIT_T) fp8_split_long_kernel(const uint16_t* __restrict__ x, int64_t ldx, int K,
                                                                uint8_t* __restrict__ xq, int64_t term_stride,
                                                                float* __restrict__ sx) {
  __shared__ float red[SPLIT_T / 64];
  const int m = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* xr = x + (int64_t)m * ldx;
  float amax = 0.f;
  for (int c = tid; c * 8 < K; c += SPLIT_T) {
    const u32x4_t v = ld_global_16(xr + c * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(bf16_bits_to_f32((v[e >> 1] >> ((e & 1) * 16)) & 0xffffu)));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  float a = red[0];
#pragma unroll
  for (int q = 1; q < SPLIT_T / 64; ++q) a = fmaxf(a, red[q]);
  int e;
  const float s = split_exponent_scale(a, &e);
  if (tid == 0) sx[m] = s;
  const float inv = ldexpf(1.f, -e);
  uint8_t* q0 = xq + (int64_t)m * K;
  for (int c = tid; c * 8 < K; c += SPLIT_T) {
    const u32x4_t v = ld_global_16(xr + c * 8);
    float f[8];
#pragma unroll
    for (int el = 0; el < 8; ++el) f[el] = bf16_bits_to_f32((v[el >> 1] >> ((el & 1) * 16)) & 0xffffu) * inv;
    uint2 hi, lo;
    split8<TERMS>(f, hi, lo);
    *reinterpret_cast<uint2*>(q0 + c * 8) = hi;
    if constexpr (TERMS == 2) *reinterpret_cast<uint2*>(q0 + term_stride + c * 8) = lo;
  }
}

template <int TERMS>
hipError_t launch_split(const LoraArgs& p, uint8_t* xq, int64_t term_stride, float* sx) {
  const auto* x = reinterpret_cast<const uint16_t*>(p.x);
  const dim3 grid((unsigned)p.M), block(SPLIT_T);
  const int64_t nch = p.K / 8;
  if (nch <= SPLIT_T * 2) fp8_split_kernel<TERMS, 2><<<grid, block, 0, p.stream>>>(x, p.ldx, (int)p.K, xq, term_stride, sx);
  else if (nch <= SPLIT_T * 8) fp8_split_kernel<TERMS, 8><<<grid, block, 0, p.stream>>>(x, p.ldx, (int)p.K, xq, term_stride, sx);
  else fp8_split_long_kernel<TERMS><<<grid, block, 0, p.stream>>>(x, p.ldx, (int)p.K, xq, term_stride, sx);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------- GEMM
template <int TERMS, bool LORA>
__global__ void __launch_bounds__(F8_NT, 1)
fp8_gemm_kernel(const uint8_t* __restrict__ xq, int64_t term_stride, const float* __restrict__ sx,
                const uint8_t* __restrict__ w, int64_t ldw, const float* __restrict__ w_scale,
                const uint16_t* __restrict__ tg, int64_t ldt, const uint16_t* __restrict__ bm, int64_t ldb,
                uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K, int r, int tiles_m, int tiles_n,
                int ge0, int ge1, int ge2, int t_gstride, RowMap wmap) {
  constexpr int STAGE = F8_TILE * (1 + TERMS);  // W tile, then the x tiles
  constexpr int OS = F8_BN * 2 + 16;            // row stride of the staged output tile
  constexpr int LDS_BYTES = (F8_S * STAGE > F8_BM * OS) ? F8_S * STAGE : F8_BM * OS;
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
  static_assert(2 * F8_BM * 128 <= LDS_BYTES, "LoRA phase fits");
  constexpr int PER_TILE = 2 * (1 + TERMS);     // fill instructions per wave per K tile
  __shared__ __attribute__((aligned(1024))) char lds[LDS_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % F8_WNW, wm = wave / F8_WNW;
  const int l32 = lane & 31, lh = lane >> 5;

  // XCD-aware grouped tile order (as the bf16 kernel)
  const int G = tiles_m * tiles_n;
  int t = blockIdx.x;
  if (G % F8_N_XCD == 0) t = (t % F8_N_XCD) * (G / F8_N_XCD) + t / F8_N_XCD;
  const int group_size = F8_GROUP_M * tiles_n;
  const int first_m = (t / group_size) * F8_GROUP_M;
  const int gm = min(tiles_m - first_m, F8_GROUP_M);
  const int tm = first_m + (t % group_size) % gm;
  const int tn = (t % group_size) / gm;
  const int m0 = tm * F8_BM, n0 = tn * F8_BN;
  if constexpr (LORA) {  // grouped launch: this tile's group takes its T column block
    const int grp = (n0 >= ge0) + (n0 >= ge1) + (n0 >= ge2);
    tg += grp * t_gstride;
  }

  // Direct-fill sources: tile base (wave-uniform) + 32-bit lane offset. Fill g of a tile
  // writes its rows 16 g .. 16 g + 15; wave v issues fills 2 v and 2 v + 1.
  const int fc = f8_fill_chunk(lane);
  const int wrow0 = wmap.P == 0 ? n0 : 0;  // mapped W rows are offsets from W's start
  uint32_t xoff[2], woff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = (wave * 2 + i) * 16 + (lane >> 2);
    xoff[i] = (uint32_t)((int64_t)(min(m0 + row, M - 1) - m0) * K + fc * 16);
    woff[i] = (uint32_t)((int64_t)(map_row(min(n0 + row, N - 1), wmap) - wrow0) * ldw + fc * 16);
  }
  const char* xbase = reinterpret_cast<const char*>(xq) + (int64_t)m0 * K;
  const char* wbase = reinterpret_cast<const char*>(w) + (int64_t)wrow0 * ldw;
  auto issue = [&](int stage, int k0) {
    char* sw = lds + stage * STAGE;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_global_load_lds(wbase + k0 + f8_opaque(woff[i]), (lds_void_t*)(sw + (wave * 2 + i) * 1024),
                                       16, 0, 0);
#pragma unroll
    for (int tt = 0; tt < TERMS; ++tt)
#pragma unroll
      for (int i = 0; i < 2; ++i)
        __builtin_amdgcn_global_load_lds(xbase + tt * term_stride + k0 + f8_opaque(xoff[i]),
                                         (lds_void_t*)(sw + (1 + tt) * F8_TILE + (wave * 2 + i) * 1024), 16, 0, 0);
  };

  f32x16_t acc[F8_NI][F8_MJ];
#pragma unroll
  for (int i = 0; i < F8_NI; ++i)
#pragma unroll
    for (int j = 0; j < F8_MJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int nk = K / F8_BK;
  // prologue: K tiles 0 and 1 in flight
  issue(0, 0);
  if (nk > 1) issue(1, F8_BK);
  for (int kt = 0; kt < nk; ++kt) {
    // tile kt has landed once at most the next tile's fills are outstanding
    if (kt + 1 < nk) f8_wait_vm<PER_TILE>();
    else f8_wait_vm<0>();
    f8_barrier();  // tile kt visible to every wave; every wave is done with tile kt - 1
    if (kt + 2 < nk) issue((kt + 2) % F8_S, (kt + 2) * F8_BK);  // into tile kt - 1's stage
    const char* sw = lds + (kt % F8_S) * STAGE;
    i32x8_t xf[TERMS][F8_MJ];
#pragma unroll
    for (int tt = 0; tt < TERMS; ++tt)
#pragma unroll
      for (int j = 0; j < F8_MJ; ++j) xf[tt][j] = f8_frag(sw + (1 + tt) * F8_TILE, wm * F8_TM + j * 32 + l32, lh);
    i32x8_t wf = f8_frag(sw, wn * F8_TN + l32, lh);
#pragma unroll
    for (int i = 0; i < F8_NI; ++i) {
      i32x8_t wn_next = wf;
      if (i + 1 < F8_NI) wn_next = f8_frag(sw, wn * F8_TN + (i + 1) * 32 + l32, lh);
#pragma unroll
      for (int tt = 0; tt < TERMS; ++tt)
#pragma unroll
        for (int j = 0; j < F8_MJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf, xf[tt][j], acc[i][j], 0, 0, 0, kE8M0One, 0,
                                                                      kE8M0One - kLoShift * tt);
      wf = wn_next;
    }
  }
  __syncthreads();  // every wave is done with the stages before the LDS is reused

  // ---- scales: 2^e[m] per token (column of the block) and w_scale[n] per channel (row)
  {
    float sm[F8_MJ];
#pragma unroll
    for (int j = 0; j < F8_MJ; ++j) sm[j] = sx[min(m0 + wm * F8_TM + j * 32 + l32, M - 1)];
#pragma unroll
    for (int i = 0; i < F8_NI; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float sc = w_scale[map_row(min(n0 + wn * F8_TN + i * 32 + g * 8 + lh * 4 + e, N - 1), wmap)];
#pragma unroll
          for (int j = 0; j < F8_MJ; ++j) acc[i][j][g * 4 + e] *= sc * sm[j];
        }
  }

  // ---- LoRA up-projection acc[n][m] += sum_j B[n][j] T[m][j], 64 ranks at a time (bf16 MFMA)
  if constexpr (LORA) {
    char* st = lds;                 // T chunk [BM m][64 ranks]
    char* sb = lds + F8_BM * 128;   // B chunk [BN n][64 ranks]
    const int nrc = (r + 63) / 64;
    for (int rc = 0; rc < nrc; ++rc) {
      const int rk0 = rc * 64;
      constexpr int CH = F8_BM * 8 / F8_NT;  // 16-byte chunks per thread
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int id = i * F8_NT + tid;
        const int row = id >> 3, c = id & 7, kr = rk0 + c * 8;
        const u32x4_t tv = (kr < r) ? ld_global_16(tg + (int64_t)min(m0 + row, M - 1) * ldt + kr) : zero_u32x4();
        const u32x4_t bv = (kr < r) ? ld_global_16(bm + (int64_t)min(n0 + row, N - 1) * ldb + kr) : zero_u32x4();
        *reinterpret_cast<u32x4_t*>(st + b16_off(row, c)) = tv;
        *reinterpret_cast<u32x4_t*>(sb + b16_off(row, c)) = bv;
      }
      __syncthreads();
      const int rem = r - rk0;
      const int nkk = rem >= 64 ? 4 : (rem + 15) / 16;
      for (int kk = 0; kk < nkk; ++kk) {
        const int c = kk * 2 + lh;
        bf16x8_t tf[F8_MJ], bf[F8_NI];
#pragma unroll
        for (int j = 0; j < F8_MJ; ++j)
          tf[j] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(st + b16_off(wm * F8_TM + j * 32 + l32, c)));
#pragma unroll
        for (int i = 0; i < F8_NI; ++i)
          bf[i] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(sb + b16_off(wn * F8_TN + i * 32 + l32, c)));
#pragma unroll
        for (int i = 0; i < F8_NI; ++i)
#pragma unroll
          for (int j = 0; j < F8_MJ; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[i], tf[j], acc[i][j], 0, 0, 0);
      }
      __syncthreads();
    }
  }

  // ---- store through LDS, whole rows (as the bf16 kernel)
  char* ot = lds;
#pragma unroll
  for (int j = 0; j < F8_MJ; ++j) {
    const int mr = wm * F8_TM + j * 32 + l32;
#pragma unroll
    for (int i = 0; i < F8_NI; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int nc = wn * F8_TN + i * 32 + g * 8 + lh * 4;
        uint2 v;
        v.x = pack_bf16x2(acc[i][j][g * 4 + 0], acc[i][j][g * 4 + 1]);
        v.y = pack_bf16x2(acc[i][j][g * 4 + 2], acc[i][j][g * 4 + 3]);
        *reinterpret_cast<uint2*>(ot + mr * OS + nc * 2) = v;
      }
  }
  __syncthreads();
  constexpr int CPR = F8_BN / 8;
  const bool a16 = ((reinterpret_cast<uintptr_t>(y) & 15u) == 0) && ((ldy & 7) == 0);
  if (a16 && m0 + F8_BM <= M && n0 + F8_BN <= N) {
    constexpr int IT = F8_BM * CPR / F8_NT;
    u32x4_t v[IT];
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int q = i * F8_NT + tid;
      v[i] = *reinterpret_cast<const u32x4_t*>(ot + (q / CPR) * OS + (q % CPR) * 16);
    }
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int q = i * F8_NT + tid;
      __builtin_nontemporal_store(v[i], reinterpret_cast<u32x4_t*>(y + (int64_t)(m0 + q / CPR) * ldy + n0 + (q % CPR) * 8));
    }
    return;
  }
  for (int q = tid; q < F8_BM * CPR; q += F8_NT) {
    const int row = q / CPR, c = q % CPR;
    const int m = m0 + row, n = n0 + c * 8;
    if (m >= M || n >= N) continue;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ot + row * OS + c * 16);
    uint16_t* dst = y + (int64_t)m * ldy + n;
    if (n + 8 <= N && a16) {
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(dst));
    } else {
      for (int e = 0; e < 8 && n + e < N; ++e) dst[e] = (uint16_t)(v[e >> 1] >> ((e & 1) * 16));
    }
  }
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

int group_end_f8(const LoraArgs& p, int g) { return g + 1 < p.groups ? (int)p.gend[g] : INT_MAX; }

}  // namespace

// The fp8 matrix-core path: fp8 W, K a multiple of 64 with 32-bit lane offsets, 16-byte
// aligned rows, groups (if any) on whole 256-wide tiles.
bool prefill_fp8_supported(const LoraArgs& p) {
  if (p.w == nullptr || p.w_dtype != kFP8) return false;
  if (p.M <= kDecodeMaxM || p.K % F8_BK != 0 || p.r % 8 != 0) return false;
  if (p.r > 0 && ((reinterpret_cast<uintptr_t>(p.b) & 15u) != 0 || p.ldb % 8 != 0)) return false;
  if ((reinterpret_cast<uintptr_t>(p.w) & 15u) != 0 || p.ldw % 16 != 0) return false;
  if (p.ldw * (int64_t)F8_BN >= ((int64_t)1 << 32) || p.K * (int64_t)F8_BM >= ((int64_t)1 << 32)) return false;
  if (p.wmap.P != 0 && p.wrows * p.ldw >= ((int64_t)1 << 32)) return false;
  if ((reinterpret_cast<uintptr_t>(p.x) & 15u) != 0 || p.ldx % 8 != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.y) & 7u) != 0 || p.ldy % 4 != 0) return false;
  for (int g = 0; g + 1 < p.groups; ++g)
    if (p.gend[g] % F8_BN != 0) return false;
  return true;
}

// Workspace after the rank pre-pass region: the activation codes [terms][M][K] and the
// per-token scales [M] fp32.
size_t prefill_fp8_workspace_bytes(int64_t M, int64_t K, int terms) {
  return align256((size_t)terms * M * K) + align256((size_t)M * 4);
}

hipError_t launch_prefill_fp8(const LoraArgs& p, const uint16_t* tg, int64_t ldt, void* scratch, int terms) {
  uint8_t* xq = reinterpret_cast<uint8_t*>(scratch);
  const int64_t term_stride = p.M * p.K;
  float* sx = reinterpret_cast<float*>(reinterpret_cast<char*>(scratch) + align256((size_t)terms * p.M * p.K));
  hipError_t e = terms == 2 ? launch_split<2>(p, xq, term_stride, sx) : launch_split<1>(p, xq, term_stride, sx);
  if (e != hipSuccess) return e;
  const int tiles_m = (int)((p.M + F8_BM - 1) / F8_BM), tiles_n = (int)((p.N + F8_BN - 1) / F8_BN);
  const dim3 grid((unsigned)(tiles_m * tiles_n)), block(F8_NT);
  const int tgs = (p.groups > 1 && tg != nullptr) ? (int)p.r : 0;
  const auto* w8 = reinterpret_cast<const uint8_t*>(p.w);
  const auto* b = reinterpret_cast<const uint16_t*>(p.b);
  auto* y = reinterpret_cast<uint16_t*>(p.y);
  const int g0 = group_end_f8(p, 0), g1 = group_end_f8(p, 1), g2 = group_end_f8(p, 2);
  const bool lora = tg != nullptr && p.r > 0;
  if (terms == 2) {
    if (lora)
      fp8_gemm_kernel<2, true><<<grid, block, 0, p.stream>>>(xq, term_stride, sx, w8, p.ldw, p.w_scale, tg, ldt, b,
                                                            p.ldb, y, p.ldy, (int)p.M, (int)p.N, (int)p.K, (int)p.r,
                                                            tiles_m, tiles_n, g0, g1, g2, tgs, p.wmap);
    else
      fp8_gemm_kernel<2, false><<<grid, block, 0, p.stream>>>(xq, term_stride, sx, w8, p.ldw, p.w_scale, tg, ldt, b,
                                                             p.ldb, y, p.ldy, (int)p.M, (int)p.N, (int)p.K, 0,
                                                             tiles_m, tiles_n, g0, g1, g2, 0, p.wmap);
  } else {
    if (lora)
      fp8_gemm_kernel<1, true><<<grid, block, 0, p.stream>>>(xq, term_stride, sx, w8, p.ldw, p.w_scale, tg, ldt, b,
                                                            p.ldb, y, p.ldy, (int)p.M, (int)p.N, (int)p.K, (int)p.r,
                                                            tiles_m, tiles_n, g0, g1, g2, tgs, p.wmap);
    else
      fp8_gemm_kernel<1, false><<<grid, block, 0, p.stream>>>(xq, term_stride, sx, w8, p.ldw, p.w_scale, tg, ldt, b,
                                                             p.ldb, y, p.ldy, (int)p.M, (int)p.N, (int)p.K, 0,
                                                             tiles_m, tiles_n, g0, g1, g2, 0, p.wmap);
  }
  return hipGetLastError();
}

}  // namespace wsl
