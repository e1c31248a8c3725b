// Decode-shaped (M <= 64 tokens) fused LoRA linear for gfx950.
//
// At small M a projection is a stream over W (N*K elements); the MFMA units are nearly
// idle and the design goal is HBM bandwidth. Launches:
//
//  K0  P_T[s][m][j] = x[m] . A[j] over K slice s           (the r rows of A)
//  K1  y[m][n] = bf16(w_scale[n] * x[m] . W[n] + T[m] . B[n])  (the N rows of W)
//      with T[m][j] = bf16(s * sum_s P_T[s][m][j])
//  K2  only when K1 splits K: sums K1's fp32 partials and finishes the rows as above.
//
// K0 and K1 are one row-group kernel: a workgroup (8 waves) owns 16*NR rows and one K
// slice; each lane streams 64 contiguous bytes of a row per step (16 rows x 4 lane
// groups per wave, waves interleaved over K), the slice of x is staged in LDS (only
// the M real rows, plus one zero row that stands in for the MFMA padding), and
// v_mfma_f32_16x16x32_bf16 forms the dot products. Wave partial sums are reduced
// through LDS. K is split only as far as the x slice must fit the 160 KB LDS; the
// partial sums of a split then go through K2 instead of any cross-workgroup hand-off
// (a device-scope fence on this part writes back and invalidates a whole XCD's L2).
//
// fp8 base rows are decoded to bf16 in registers (v_cvt_pk_f32_fp8). Reference
// arithmetic: the decode loop runs the same projections at small M
// (scripts/generate/_generation.py:35-80 calling
// torchtitan/models/llama3/model/model.py:189-192,392-398).
#include "wsl_common.h"

namespace wsl {
namespace {

constexpr int DT = 512;                   // threads per streaming workgroup (8 waves)
constexpr int NWV = DT / 64;
constexpr int64_t LDS_MAX = 160 * 1024;   // gfx950 LDS per workgroup
constexpr int64_t XS_MAX = LDS_MAX - 16 * 1024;  // x slice budget (rest: reduction)
constexpr int RT = 256;                   // threads of the reduce kernel

// Elements of K one lane covers per step (64 bytes of the row) and per wave step.
template <int WDT> struct Geo {
  static constexpr int LANE_K = (WDT == kFP8) ? 64 : 32;
  static constexpr int WAVE_K = 4 * LANE_K;  // 4 lane groups
};

// x slice staged in LDS: rows 0..M-1 of x, then one zero row (index M) read by the
// MFMA lanes of padding columns; row stride kc*2 + 16 bytes (bank spread).
__device__ __forceinline__ int xs_row(int m, int M) { return m < M ? m : M; }
__device__ __forceinline__ int xs_off(int row, int k, int xs_stride) { return row * xs_stride + k * 2; }

// One row group (NR blocks of 16 rows) of a [rows, K] bf16/fp8 matrix against x^T over
// the local K range [0, kc) starting at global column kbeg.
template <int WDT, int NR, int MB>
__device__ __forceinline__ void row_group_dot(const void* __restrict__ wmat, int64_t ldw, int rows,
                                              int row0, int kbeg, int kc, int M, const char* xs,
                                              int xs_stride, f32x4_t (&acc)[NR][MB]) {
  using G = Geo<WDT>;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int l16 = lane & 15;
  const int grp = lane >> 4;
  const int nsteps = kc / G::WAVE_K;

  int64_t rowoff[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int rr = row0 + i * 16 + l16;
    rowoff[i] = (int64_t)(rr < rows ? rr : rows - 1) * ldw;
  }
  int xrow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) xrow[mb] = xs_row(mb * 16 + l16, M);

  for (int st = wave; st < nsteps; st += NWV) {
    const int kl = st * G::WAVE_K + grp * G::LANE_K;  // local k of this lane's run
    const int kg = kbeg + kl;
    u32x4_t wv[NR][4];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if constexpr (WDT == kBF16) {
          wv[i][u] = ld_global_16(reinterpret_cast<const uint16_t*>(wmat) + rowoff[i] + kg + u * 8);
        } else {
          wv[i][u] = ld_global_16(reinterpret_cast<const uint8_t*>(wmat) + rowoff[i] + kg + u * 16);
        }
      }
    }
    if constexpr (WDT == kBF16) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        bf16x8_t xf[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          xf[mb] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(xs + xs_off(xrow[mb], kl + u * 8, xs_stride)));
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
            xf[mb] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(xs + xs_off(xrow[mb], kl + u * 16 + h * 8, xs_stride)));
#pragma unroll
          for (int i = 0; i < NR; ++i) {
            const u32x4_t wb = fp8x8_to_bf16x8(wv[i][u][2 * h], wv[i][u][2 * h + 1]);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
              acc[i][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wb), xf[mb], acc[i][mb], 0, 0, 0);
          }
        }
      }
    }
  }
}

// Role of a streaming launch.
enum Role : int { kRoleT = 0, kRoleY = 1, kRolePartial = 2 };

struct DecodeArgs {
  const uint16_t* x; int64_t ldx;
  const void* mat; int64_t ldm;    // A (role T) or W (roles Y, partial)
  int rows;                        // r or N
  int M, kc;
  float* part;                     // role T / partial: [splits][M][rows] fp32 sums
  // finishing (role Y and the reduce kernel):
  const float* tpart; int tsplits; // K0's partials [tsplits][M][r]
  float s;                         // LoRA scale
  const float* w_scale;
  const uint16_t* b; int64_t ldb; int r;
  uint16_t* y; int64_t ldy;
};

// T[m][j] = bf16(s * sum_s P_T[s][m][j]) into LDS (fp32 values), m < M, j < r.
__device__ __forceinline__ void load_t(const DecodeArgs& p, float* tl, int nthreads) {
  for (int q = threadIdx.x; q < p.M * p.r; q += nthreads) {
    float v = 0.f;
    for (int sp = 0; sp < p.tsplits; ++sp) v += p.tpart[(int64_t)sp * p.M * p.r + q];
    tl[q] = bf16_bits_to_f32(f32_to_bf16_bits(p.s * v));
  }
}

// y[m][row] = bf16(w_scale[row] * v + T[m] . B[row]); tr is the row T[m] (fp32 values).
__device__ __forceinline__ void finish_one(const DecodeArgs& p, const float* tr, int m, int row, float v) {
  float out = (p.w_scale != nullptr) ? v * p.w_scale[row] : v;
  if (p.r > 0) {
    const uint16_t* br = p.b + (int64_t)row * p.ldb;
    for (int j0 = 0; j0 < p.r; j0 += 8) {
      const u32x4_t bv = ld_global_16(br + j0);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        out += tr[j0 + 2 * q] * bf16_bits_to_f32(bv[q] & 0xffffu);
        out += tr[j0 + 2 * q + 1] * bf16_bits_to_f32(bv[q] >> 16);
      }
    }
  }
  p.y[(int64_t)m * p.ldy + row] = f32_to_bf16_bits(out);
}

template <int WDT, int NR, int MB, int ROLE>
__global__ void __launch_bounds__(DT)
stream_kernel(DecodeArgs p) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int ROWS = 16 * NR;
  constexpr int MC = 16 * MB;
  constexpr int PER_LANE = NR * MB * 4;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = blockIdx.x;
  const int ks = blockIdx.y;
  const int kbeg = ks * p.kc;
  const int row0 = g * ROWS;
  const int xs_stride = p.kc * 2 + 16;
  char* xs = smem;

  // Stage x[0..M)[kbeg .. kbeg+kc) and the zero row M.
  const int chunks_per_row = p.kc / 8;
  const int nchunks = (p.M + 1) * chunks_per_row;
  for (int c = tid; c < nchunks; c += DT) {
    const int m = c / chunks_per_row;
    const int kk = (c % chunks_per_row) * 8;
    const u32x4_t v = (m < p.M) ? ld_global_16(p.x + (int64_t)m * p.ldx + kbeg + kk) : zero_u32x4();
    *reinterpret_cast<u32x4_t*>(xs + xs_off(m, kk, xs_stride)) = v;
  }
  __syncthreads();

  f32x4_t acc[NR][MB];
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[i][mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  row_group_dot<WDT, NR, MB>(p.mat, p.ldm, p.rows, row0, kbeg, p.kc, p.M, xs, xs_stride, acc);

  // Cross-wave reduction through LDS into sums[row][m] (fp32, ROWS x MC).
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
  float* sums = red + (NWV - 1) * PER_LANE * 64;
  float* tl = sums + ROWS * MC;  // T [M][r] (role Y)
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
#pragma unroll
    for (int i = 0; i < NR; ++i) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        f32x4_t v = acc[i][mb];
        for (int wv = 0; wv < NWV - 1; ++wv)
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] += red[(wv * PER_LANE + (i * MB + mb) * 4 + e) * 64 + lane];
        // D[row][m]: lane holds m = l16, rows grp*4 + e of block i
#pragma unroll
        for (int e = 0; e < 4; ++e) sums[(i * 16 + grp * 4 + e) * MC + mb * 16 + l16] = v[e];
      }
    }
  }
  if constexpr (ROLE == kRoleY) load_t(p, tl, DT);
  __syncthreads();

  const int nrow = min(ROWS, p.rows - row0);
  for (int q = tid; q < nrow * p.M; q += DT) {
    const int m = q / nrow, rl = q % nrow;
    const float v = sums[rl * MC + m];
    if constexpr (ROLE == kRoleY) {
      finish_one(p, tl + m * p.r, m, row0 + rl, v);
    } else {
      p.part[((int64_t)ks * p.M + m) * p.rows + row0 + rl] = v;
    }
  }
}

// K2: y = bf16(w_scale * sum_s P[s] + T . B^T); one thread per (m, n), blockIdx.y = m.
__global__ void __launch_bounds__(RT) reduce_kernel(DecodeArgs p, int splits) {
  __shared__ float tl[256];  // T[m][0..r), r <= 256
  const int m = blockIdx.y;
  for (int j = threadIdx.x; j < p.r; j += RT) {
    float v = 0.f;
    for (int sp = 0; sp < p.tsplits; ++sp) v += p.tpart[((int64_t)sp * p.M + m) * p.r + j];
    tl[j] = bf16_bits_to_f32(f32_to_bf16_bits(p.s * v));
  }
  __syncthreads();
  const int n = blockIdx.x * RT + threadIdx.x;
  if (n >= p.rows) return;
  float v = 0.f;
  for (int sp = 0; sp < splits; ++sp) v += p.part[((int64_t)sp * p.M + m) * p.rows + n];
  finish_one(p, tl, m, n, v);
}

struct Split {
  int splits, kc, groups;
};

int wave_k_of(int wdt) { return wdt == kFP8 ? 256 : 128; }

int64_t xs_bytes(int64_t M, int64_t kc) { return (M + 1) * (kc * 2 + 16); }

// The smallest K split whose x slice fits the LDS budget (each slice a whole number of
// wave steps).
Split plan_split(int64_t rows, int64_t K, int64_t M, int nr, int wdt) {
  Split sp;
  sp.groups = (int)((rows + 16 * nr - 1) / (16 * nr));
  const int wk = wave_k_of(wdt);
  int64_t s = 1;
  while (xs_bytes(M, K / s) > XS_MAX && K % (s * 2 * wk) == 0) s *= 2;
  sp.splits = (int)s;
  sp.kc = (int)(K / s);
  return sp;
}

struct DecodePlan {
  int mb, nr;
  Split t, y;
  size_t off_pt, off_py, total;
};

DecodePlan plan_decode(int64_t M, int64_t N, int64_t K, int64_t r, int wdt) {
  DecodePlan pl;
  pl.mb = (int)((M + 15) / 16);
  if (pl.mb < 1) pl.mb = 1;
  pl.nr = pl.mb >= 3 ? 2 : 1;
  pl.y = plan_split(N, K, M, pl.nr, wdt);
  if (r > 0) pl.t = plan_split(r, K, M, 1, kBF16);
  else pl.t = Split{1, (int)K, 0};
  size_t off = kCounterBytes;  // the decode path keeps no counters; the prefix is reserved
  pl.off_pt = off;
  off += (size_t)pl.t.splits * M * r * 4;
  off = (off + 255) & ~(size_t)255;
  pl.off_py = off;
  if (pl.y.splits > 1) off += (size_t)pl.y.splits * M * N * 4;
  pl.total = off;
  return pl;
}

size_t stream_smem(int64_t M, int kc, int nr, int mb, int r) {
  const size_t xs = (size_t)xs_bytes(M, kc);
  const size_t red = (size_t)((NWV - 1) * nr * mb * 4 * 64 + 16 * nr * 16 * mb + M * r) * 4;
  return xs > red ? xs : red;
}

bool plan_ok(const DecodePlan& pl, int64_t M, int64_t r) {
  if (xs_bytes(M, pl.y.kc) > XS_MAX) return false;
  if (pl.t.groups > 0 && xs_bytes(M, pl.t.kc) > XS_MAX) return false;
  return stream_smem(M, pl.y.kc, pl.nr, pl.mb, (int)r) <= (size_t)LDS_MAX &&
         (size_t)M * r * 4 <= 65536;
}

template <class KernelT>
void allow_lds(KernelT kernel) {
  // Raise the dynamic LDS limit of this kernel to the gfx950 maximum (idempotent).
  (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_MAX);
}

template <int WDT, int NR, int MB, int ROLE>
hipError_t launch_stream(const DecodeArgs& a, int groups, int splits, int r, hipStream_t st) {
  static bool ready = false;  // set once per instantiation; the attribute is per kernel
  if (!ready) {
    allow_lds(stream_kernel<WDT, NR, MB, ROLE>);
    ready = true;
  }
  const size_t sm = stream_smem(a.M, a.kc, NR, MB, r);
  stream_kernel<WDT, NR, MB, ROLE><<<dim3((unsigned)groups, (unsigned)splits), dim3(DT), sm, st>>>(a);
  return hipGetLastError();
}

template <int WDT, int ROLE>
hipError_t dispatch(const DecodeArgs& a, int mb, int nr, int groups, int splits, int r, hipStream_t st) {
  if (nr == 1) {
    switch (mb) {
      case 1: return launch_stream<WDT, 1, 1, ROLE>(a, groups, splits, r, st);
      case 2: return launch_stream<WDT, 1, 2, ROLE>(a, groups, splits, r, st);
      case 3: return launch_stream<WDT, 1, 3, ROLE>(a, groups, splits, r, st);
      default: return launch_stream<WDT, 1, 4, ROLE>(a, groups, splits, r, st);
    }
  }
  switch (mb) {
    case 1: return launch_stream<WDT, 2, 1, ROLE>(a, groups, splits, r, st);
    case 2: return launch_stream<WDT, 2, 2, ROLE>(a, groups, splits, r, st);
    case 3: return launch_stream<WDT, 2, 3, ROLE>(a, groups, splits, r, st);
    default: return launch_stream<WDT, 2, 4, ROLE>(a, groups, splits, r, st);
  }
}

bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

}  // namespace

bool decode_supported(const LoraArgs& p) {
  if (p.M < 1 || p.M > kDecodeMaxM) return false;
  if (p.w == nullptr) return false;  // the delta-only form runs on the prefill path
  if (p.N > (int64_t)1 << 30 || p.K > (int64_t)1 << 30) return false;
  const bool fp8 = p.w_dtype == kFP8;
  if (p.K % wave_k_of(p.w_dtype) != 0) return false;
  if (!aligned16(p.x) || p.ldx % 8 != 0) return false;
  if (!aligned16(p.w) || p.ldw % (fp8 ? 16 : 8) != 0) return false;
  if (p.r > 0) {
    if (p.r % 8 != 0) return false;
    if (!aligned16(p.a) || p.lda % 8 != 0) return false;
    if (!aligned16(p.b) || p.ldb % 8 != 0) return false;
  }
  return plan_ok(plan_decode(p.M, p.N, p.K, p.r, p.w_dtype), p.M, p.r);
}

size_t decode_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, int w_dtype) {
  return plan_decode(M, N, K, r, w_dtype).total;
}

hipError_t launch_decode(const LoraArgs& p) {
  const DecodePlan pl = plan_decode(p.M, p.N, p.K, p.r, p.w_dtype);
  char* ws = reinterpret_cast<char*>(p.ws);
  float* tpart = reinterpret_cast<float*>(ws + pl.off_pt);
  if (p.r > 0) {
    DecodeArgs t{};
    t.x = reinterpret_cast<const uint16_t*>(p.x); t.ldx = p.ldx;
    t.mat = p.a; t.ldm = p.lda; t.rows = (int)p.r;
    t.M = (int)p.M; t.kc = pl.t.kc;
    t.part = tpart;
    hipError_t e = dispatch<kBF16, kRoleT>(t, pl.mb, 1, pl.t.groups, pl.t.splits, 0, p.stream);
    if (e != hipSuccess) return e;
  }
  DecodeArgs y{};
  y.x = reinterpret_cast<const uint16_t*>(p.x); y.ldx = p.ldx;
  y.mat = p.w; y.ldm = p.ldw; y.rows = (int)p.N;
  y.M = (int)p.M; y.kc = pl.y.kc;
  y.part = reinterpret_cast<float*>(ws + pl.off_py);
  y.tpart = tpart; y.tsplits = pl.t.splits; y.s = p.scale;
  y.w_scale = p.w_scale;
  y.b = reinterpret_cast<const uint16_t*>(p.b); y.ldb = p.ldb; y.r = (int)p.r;
  y.y = reinterpret_cast<uint16_t*>(p.y); y.ldy = p.ldy;
  const bool fp8 = p.w_dtype == kFP8;
  const int r = (int)p.r;
  if (pl.y.splits == 1) {
    return fp8 ? dispatch<kFP8, kRoleY>(y, pl.mb, pl.nr, pl.y.groups, 1, r, p.stream)
               : dispatch<kBF16, kRoleY>(y, pl.mb, pl.nr, pl.y.groups, 1, r, p.stream);
  }
  hipError_t e = fp8 ? dispatch<kFP8, kRolePartial>(y, pl.mb, pl.nr, pl.y.groups, pl.y.splits, 0, p.stream)
                     : dispatch<kBF16, kRolePartial>(y, pl.mb, pl.nr, pl.y.groups, pl.y.splits, 0, p.stream);
  if (e != hipSuccess) return e;
  reduce_kernel<<<dim3((unsigned)((p.N + RT - 1) / RT), (unsigned)p.M), dim3(RT), 0, p.stream>>>(y, pl.y.splits);
  return hipGetLastError();
}

}  // namespace wsl
