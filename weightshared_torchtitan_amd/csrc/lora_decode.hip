// Decode-shaped (M <= 64 tokens) fused LoRA linear for gfx950.
//
// At small M the projection is a stream over W (N*K elements) and the MFMA units are
// nearly idle, so the design goal is HBM bandwidth:
//
//  1. skinny_partial: grid = (row groups of [W ; A], K splits). The rows of the
//     LoRA down-projection A [r,K] are appended after the N rows of W, so x . A^T is
//     produced by the same launch that streams W. Each lane streams 64 contiguous
//     bytes of one W row per step (16 rows x 4 lane groups per wave), x comes from
//     LDS, and v_mfma_f32_16x16x32_bf16 does the dot products (M padded to 16).
//     The 4 waves of a workgroup split its K range; their partial sums are reduced
//     through LDS and written as fp32 partials P[split][m][row].
//  2. skinny_epilogue: y[m][n] = bf16(w_scale[n] * sum_s P[s][m][n] + T[m] . B[n]),
//     T[m][j] = bf16(s * sum_s P[s][m][N + j]).
//
// fp8 base rows are decoded to bf16 in registers (v_cvt_pk_f32_fp8); the per-channel
// scale is applied in the epilogue. Reference arithmetic: the decode loop runs the
// same projections at small M (scripts/generate/_generation.py:35-80 calling
// torchtitan/models/llama3/model/model.py:189-192,392-398).
#include "wsl_common.h"

namespace wsl {
namespace {

constexpr int DT = 256;            // threads per workgroup (4 waves)
constexpr int XS_MAX_BYTES = 65536;  // LDS budget for the staged x slice

// Elements of K one lane covers per step (64 bytes of W) and per wave step.
template <int WDT> struct Geo {
  static constexpr int LANE_K = (WDT == kFP8) ? 64 : 32;
  static constexpr int WAVE_K = 4 * LANE_K;  // 4 lane groups
};

// x slice [M][kc] staged in LDS with a 16-byte row pad (row stride = kc*2 + 16).
__device__ __forceinline__ int xs_off(int m, int k, int xs_stride) { return m * xs_stride + k * 2; }

// One row group (NR blocks of 16 rows) of a [rows, K] bf16/fp8 matrix against x^T.
template <int WDT, int NR, int MB>
__device__ __forceinline__ void row_group_dot(const void* __restrict__ wmat, int64_t ldw, int rows,
                                              int row0, int kbeg, int kc, const char* xs,
                                              int xs_stride, f32x4_t (&acc)[NR][MB]) {
  using G = Geo<WDT>;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int l16 = lane & 15;
  const int grp = lane >> 4;
  const int nsteps = kc / G::WAVE_K;

  int rowp[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    int rr = row0 + i * 16 + l16;
    rowp[i] = rr < rows ? rr : rows - 1;
  }

  for (int st = wave; st < nsteps; st += 4) {
    const int kl = st * G::WAVE_K + grp * G::LANE_K;  // local k of this lane's run
    const int kg = kbeg + kl;
    u32x4_t wv[NR][4];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if constexpr (WDT == kBF16) {
          wv[i][u] = ld_global_16(reinterpret_cast<const uint16_t*>(wmat) + (int64_t)rowp[i] * ldw + kg + u * 8);
        } else {
          wv[i][u] = ld_global_16(reinterpret_cast<const uint8_t*>(wmat) + (int64_t)rowp[i] * ldw + kg + u * 16);
        }
      }
    }
    if constexpr (WDT == kBF16) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        bf16x8_t xf[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          xf[mb] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(xs + xs_off(mb * 16 + l16, kl + u * 8, xs_stride)));
#pragma unroll
        for (int i = 0; i < NR; ++i)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
            acc[i][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wv[i][u]), xf[mb], acc[i][mb], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          bf16x8_t xf[MB];
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
            xf[mb] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(
                xs + xs_off(mb * 16 + l16, kl + u * 16 + h * 8, xs_stride)));
#pragma unroll
          for (int i = 0; i < NR; ++i) {
            u32x4_t wb = fp8x8_to_bf16x8(wv[i][u][2 * h], wv[i][u][2 * h + 1]);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
              acc[i][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wb), xf[mb], acc[i][mb], 0, 0, 0);
          }
        }
      }
    }
  }
}

template <int WDT, int NR, int MB>
__global__ void __launch_bounds__(DT)
skinny_partial(const uint16_t* __restrict__ x, int64_t ldx,
               const void* __restrict__ w, int64_t ldw,
               const uint16_t* __restrict__ a, int64_t lda,
               float* __restrict__ part, int M, int N, int K, int r, int kc, int groups_w,
               const float* __restrict__ w_scale, uint16_t* __restrict__ ydir, int64_t ldy) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int ks = blockIdx.y;
  const int kbeg = ks * kc;
  const int xs_stride = kc * 2 + 16;
  char* xs = smem;

  // Stage x[0..16*MB)[kbeg .. kbeg+kc) (rows >= M zero-filled).
  const int chunks_per_row = kc / 8;
  const int nchunks = 16 * MB * chunks_per_row;
  for (int c = tid; c < nchunks; c += DT) {
    int m = c / chunks_per_row;
    int kk = (c % chunks_per_row) * 8;
    u32x4_t v = (m < M) ? ld_global_16(x + (int64_t)m * ldx + kbeg + kk) : zero_u32x4();
    *reinterpret_cast<u32x4_t*>(xs + xs_off(m, kk, xs_stride)) = v;
  }
  __syncthreads();

  f32x4_t acc[NR][MB];
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[i][mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int g = blockIdx.x;
  int row0, rows, col0;
  if (g < groups_w) {
    row0 = g * NR * 16;
    rows = N;
    col0 = 0;
    row_group_dot<WDT, NR, MB>(w, ldw, N, row0, kbeg, kc, xs, xs_stride, acc);
  } else {
    row0 = (g - groups_w) * NR * 16;
    rows = r;
    col0 = N;
    row_group_dot<kBF16, NR, MB>(a, lda, r, row0, kbeg, kc, xs, xs_stride, acc);
  }

  // Cross-wave reduction through LDS (reusing the x slice after a barrier).
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
  constexpr int PER_LANE = NR * MB * 4;
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < NR; ++i)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          red[((wave - 1) * PER_LANE + (i * MB + mb) * 4 + e) * 64 + lane] = acc[i][mb][e];
  }
  __syncthreads();
  if (wave == 0) {
    const int l16 = lane & 15;
    const int grp = lane >> 4;
    const int ncols = N + r;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        f32x4_t v = acc[i][mb];
#pragma unroll
        for (int wv = 0; wv < 3; ++wv)
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] += red[(wv * PER_LANE + (i * MB + mb) * 4 + e) * 64 + lane];
        // D[n][m]: lane holds m = l16, n = grp*4 + e
        const int m = mb * 16 + l16;
        const int rr = row0 + i * 16 + grp * 4;
        if (m < M) {
          if (ydir != nullptr) {
            // r = 0 and one split: finish here (dequantisation scale, bf16 store).
            uint16_t* dst = ydir + (int64_t)m * ldy + rr;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (rr + e < rows) dst[e] = f32_to_bf16_bits(w_scale != nullptr ? v[e] * w_scale[rr + e] : v[e]);
          } else {
            float* dst = part + ((int64_t)ks * M + m) * ncols + col0 + rr;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (rr + e < rows) dst[e] = v[e];
          }
        }
      }
    }
  }
}

// y[m][n] = bf16(w_scale[n] * sum_s P[s][m][n] + sum_j T[m][j] * B[n][j])
template <int MB>
__global__ void __launch_bounds__(DT)
skinny_epilogue(const float* __restrict__ part, int splits, const float* __restrict__ w_scale,
                const uint16_t* __restrict__ b, int64_t ldb, float s, bool has_w,
                uint16_t* __restrict__ y, int64_t ldy, int M, int N, int r) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  float* tl = reinterpret_cast<float*>(smem);  // T [M][r] (bf16-rounded values)
  const int ncols = N + r;
  for (int idx = threadIdx.x; idx < M * r; idx += DT) {
    int m = idx / r, j = idx % r;
    float t = 0.f;
    for (int sp = 0; sp < splits; ++sp) t += part[((int64_t)sp * M + m) * ncols + N + j];
    tl[idx] = bf16_bits_to_f32(f32_to_bf16_bits(s * t));
  }
  __syncthreads();
  const int n = blockIdx.x * DT + threadIdx.x;
  if (n >= N) return;
  float acc[16 * MB];
  const float sc = (w_scale != nullptr) ? w_scale[n] : 1.f;
#pragma unroll
  for (int m = 0; m < 16 * MB; ++m) {
    float v = 0.f;
    if (has_w && m < M)
      for (int sp = 0; sp < splits; ++sp) v += part[((int64_t)sp * M + m) * ncols + n];
    acc[m] = v * sc;
  }
  const uint16_t* br = b + (int64_t)n * ldb;
  for (int j0 = 0; j0 < r; j0 += 8) {
    u32x4_t bv = ld_global_16(br + j0);
    float bf[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      bf[2 * q] = bf16_bits_to_f32(bv[q] & 0xffffu);
      bf[2 * q + 1] = bf16_bits_to_f32(bv[q] >> 16);
    }
#pragma unroll
    for (int m = 0; m < 16 * MB; ++m) {
      if (m < M) {
        const float* tr = tl + m * r + j0;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m] += tr[e] * bf[e];
      }
    }
  }
#pragma unroll
  for (int m = 0; m < 16 * MB; ++m)
    if (m < M) y[(int64_t)m * ldy + n] = f32_to_bf16_bits(acc[m]);
}

struct DecodePlan {
  int mb, nr, splits, kc, groups_w, groups_a;
};

int wave_k_of(int w_dtype, bool has_w) { return (w_dtype == kFP8 && has_w) ? 256 : 128; }

bool xs_fits(int mb, int64_t kc) { return (int64_t)16 * mb * (kc * 2 + 16) <= XS_MAX_BYTES; }

// Split K until (a) the staged x slice fits the LDS budget and (b) the grid covers the
// 256 CUs twice, keeping every split a whole number of wave steps.
DecodePlan plan_decode(int64_t M, int64_t N, int64_t K, int64_t r, int w_dtype, bool has_w) {
  DecodePlan pl;
  pl.mb = (int)((M + 15) / 16);
  if (pl.mb < 1) pl.mb = 1;
  pl.nr = pl.mb >= 3 ? 4 : (pl.mb == 2 ? 2 : 1);
  const int wk = wave_k_of(w_dtype, has_w);
  pl.groups_w = has_w ? (int)((N + 16 * pl.nr - 1) / (16 * pl.nr)) : 0;
  pl.groups_a = (int)((r + 16 * pl.nr - 1) / (16 * pl.nr));
  const int64_t groups = pl.groups_w + pl.groups_a;
  int64_t s = 1;
  while ((!xs_fits(pl.mb, K / s) || groups * s < 512) && K % (s * 2 * wk) == 0 && s < 64) s *= 2;
  pl.splits = (int)s;
  pl.kc = (int)(K / s);
  return pl;
}

bool plan_ok(const DecodePlan& pl) { return xs_fits(pl.mb, pl.kc); }

size_t smem_partial_bytes(const DecodePlan& pl) {
  size_t xs = (size_t)16 * pl.mb * (pl.kc * 2 + 16);
  size_t red = (size_t)3 * pl.nr * pl.mb * 4 * 64 * 4;
  return xs > red ? xs : red;
}

template <int WDT, int NR, int MB>
hipError_t launch_partial(const LoraArgs& p, const DecodePlan& pl, float* part, bool direct) {
  dim3 grid((unsigned)(pl.groups_w + pl.groups_a), (unsigned)pl.splits);
  size_t sm = smem_partial_bytes(pl);
  skinny_partial<WDT, NR, MB><<<grid, dim3(DT), sm, p.stream>>>(
      reinterpret_cast<const uint16_t*>(p.x), p.ldx, p.w, p.ldw,
      reinterpret_cast<const uint16_t*>(p.a), p.lda, part, (int)p.M, (int)p.N, (int)p.K,
      (int)p.r, pl.kc, pl.groups_w, p.w_scale, direct ? reinterpret_cast<uint16_t*>(p.y) : nullptr,
      p.ldy);
  return hipGetLastError();
}

template <int WDT>
hipError_t dispatch_partial(const LoraArgs& p, const DecodePlan& pl, float* part, bool direct) {
  switch (pl.mb) {
    case 1: return launch_partial<WDT, 1, 1>(p, pl, part, direct);
    case 2: return launch_partial<WDT, 2, 2>(p, pl, part, direct);
    case 3: return launch_partial<WDT, 4, 3>(p, pl, part, direct);
    default: return launch_partial<WDT, 4, 4>(p, pl, part, direct);
  }
}

template <int MB>
hipError_t launch_epi(const LoraArgs& p, const DecodePlan& pl, const float* part) {
  dim3 grid((unsigned)((p.N + DT - 1) / DT));
  size_t sm = (size_t)p.M * p.r * 4;
  skinny_epilogue<MB><<<grid, dim3(DT), sm, p.stream>>>(
      part, pl.splits, p.w != nullptr ? p.w_scale : nullptr,
      reinterpret_cast<const uint16_t*>(p.b), p.ldb, p.scale, p.w != nullptr,
      reinterpret_cast<uint16_t*>(p.y), p.ldy, (int)p.M, (int)p.N, (int)p.r);
  return hipGetLastError();
}

bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

}  // namespace

bool decode_supported(const LoraArgs& p) {
  if (p.M < 1 || p.M > kDecodeMaxM) return false;
  if (p.N > (int64_t)1 << 30 || p.K > (int64_t)1 << 30) return false;
  const bool fp8 = p.w != nullptr && p.w_dtype == kFP8;
  if (p.K % wave_k_of(p.w_dtype, p.w != nullptr) != 0) return false;
  if (!aligned16(p.x) || p.ldx % 8 != 0) return false;
  if (p.w != nullptr && (!aligned16(p.w) || p.ldw % (fp8 ? 16 : 8) != 0)) return false;
  if (p.r > 0) {
    if (p.r % 8 != 0) return false;
    if (!aligned16(p.a) || p.lda % 8 != 0) return false;
    if (!aligned16(p.b) || p.ldb % 8 != 0) return false;
  }
  if (p.w == nullptr && p.r == 0) return false;
  const int wdt = p.w != nullptr ? p.w_dtype : kBF16;
  return plan_ok(plan_decode(p.M, p.N, p.K, p.r, wdt, p.w != nullptr));
}

size_t decode_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, int w_dtype) {
  // The launcher plans with or without a base weight; size for the larger of the two.
  DecodePlan a = plan_decode(M, N, K, r, w_dtype, true);
  DecodePlan b = plan_decode(M, N, K, r, kBF16, false);
  size_t sa = (r == 0 && a.splits == 1) ? 0 : (size_t)a.splits * M * (N + r) * 4;
  size_t sb = (size_t)b.splits * M * (N + r) * 4;
  return sa > sb ? sa : sb;
}

hipError_t launch_decode(const LoraArgs& p) {
  const bool has_w = p.w != nullptr;
  const int wdt = has_w ? p.w_dtype : kBF16;
  DecodePlan pl = plan_decode(p.M, p.N, p.K, p.r, wdt, has_w);
  float* part = reinterpret_cast<float*>(p.ws);
  const bool direct = p.r == 0 && pl.splits == 1;
  hipError_t e = (wdt == kFP8) ? dispatch_partial<kFP8>(p, pl, part, direct)
                               : dispatch_partial<kBF16>(p, pl, part, direct);
  if (e != hipSuccess || direct) return e;
  switch (pl.mb) {
    case 1: return launch_epi<1>(p, pl, part);
    case 2: return launch_epi<2>(p, pl, part);
    case 3: return launch_epi<3>(p, pl, part);
    default: return launch_epi<4>(p, pl, part);
  }
}

}  // namespace wsl
