// Prefill-shaped fused LoRA linear for gfx950 (CDNA4).
//
//   y[M,N] = (x . W^T) * diag(w_scale) + T . B^T,   T = bf16(s * x . A^T)
//
// One workgroup (4 waves, 256 threads) owns a 256(n) x 256(m) output tile; each wave
// owns 128 x 128 of it as 4 x 4 blocks of v_mfma_f32_32x32x16_bf16 (fp32 accumulate).
// K is walked in 64-wide tiles staged through swizzled, double-buffered LDS.
//
// LoRA fusion (rank r <= 64): while the x tile of a K step is LDS-resident, the same
// x fragments also feed x . A^T for the workgroup's 256 rows (the rank-r
// down-projection, computed once per workgroup, never written to HBM). After the K
// loop T is scaled, rounded to bf16 and parked in LDS, and the rank-r up-projection
// T . B^T accumulates into the same accumulator registers as x . W^T.
// For r > 64, T comes from a pre-pass kernel (workspace) and is consumed the same way.
//
// The MFMA "A" operand is the W tile (rows n) and the "B" operand the x tile (rows m),
// so each lane ends with 4 consecutive n of one m per accumulator group: the bf16
// result leaves as 8-byte stores.
//
// Reference arithmetic being fused: torchtitan/models/llama3/model/model.py:189-192
// (LoRAModule.forward), :392-398 (base projection + broadcast_add with g = 1).
#include "wsl_common.h"

namespace wsl {
namespace {

constexpr int BM = 256;   // m rows per workgroup tile
constexpr int BN = 256;   // n rows per workgroup tile
constexpr int BK = 64;    // K per LDS stage
constexpr int NT = 256;   // threads per workgroup
constexpr int RIN = 64;   // largest rank whose down-projection runs inside the kernel
constexpr int ROW_BYTES = BK * 2;                  // 128 B per LDS row (8 chunks of 16 B)
constexpr int TILE_BYTES = 256 * ROW_BYTES;        // 32 KB for a 256-row operand tile
constexpr int RANK_A_BYTES = RIN * ROW_BYTES;      // 8 KB for the rank-A K slice
constexpr int STAGE_BYTES = 2 * TILE_BYTES + RANK_A_BYTES;  // 72 KB
constexpr int LDS_BYTES = 2 * STAGE_BYTES;                  // 144 KB (gfx950: 160 KB / CU)

// Byte offset of 16-byte chunk `c` (0..7) of LDS row `row`. XOR swizzle: the 8 rows a
// group of lanes touches at one chunk index land in 8 distinct bank groups.
__device__ __forceinline__ int lds_off(int row, int c) {
  return row * ROW_BYTES + ((c ^ (row & 7)) << 4);
}

__device__ __forceinline__ u32x4_t lds_read16(const char* base, int off) {
  return *reinterpret_cast<const u32x4_t*>(base + off);
}
__device__ __forceinline__ void lds_write16(char* base, int off, u32x4_t v) {
  *reinterpret_cast<u32x4_t*>(base + off) = v;
}

template <int WDT, bool HAS_W, bool IN_T, bool GATHER>
__global__ void __launch_bounds__(NT, 1)
prefill_kernel(const uint16_t* __restrict__ x, int64_t ldx,
               const int64_t* __restrict__ gidx, int64_t grows,
               const void* __restrict__ w, int64_t ldw, const float* __restrict__ w_scale,
               const uint16_t* __restrict__ a, int64_t lda,
               const uint16_t* __restrict__ tg, int64_t ldt,
               const uint16_t* __restrict__ bm, int64_t ldb, float s,
               uint16_t* __restrict__ y, int64_t ldy,
               int M, int N, int K, int r, int tiles_m) {
  __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wi = wave & 1;   // n half of the tile
  const int wj = wave >> 1;  // m half of the tile
  const int l32 = lane & 31;
  const int lh = lane >> 5;

  const int tile = blockIdx.x;
  const int tm = tile % tiles_m;
  const int tn = tile / tiles_m;
  const int m0 = tm * BM;
  const int n0 = tn * BN;

  // ---- global -> register staging (8 chunks per operand tile per thread) ----
  // chunk id = i*256 + tid  ->  row = i*32 + tid/8, chunk = tid%8
  const int ld_c = tid & 7;
  const int ld_r = tid >> 3;
  u32x4_t stx[8];
  u32x4_t stw[8];
  u32x4_t sta[2];

  const int rpad32 = IN_T ? ((r + 31) & ~31) : 0;  // rank rows computed in-kernel

  auto load_stage = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int row = m0 + i * 32 + ld_r;
      row = row < M ? row : M - 1;
      if constexpr (GATHER) {
        const int64_t id = gidx[row];
        stx[i] = (id >= 0 && id < grows) ? ld_global_16(x + id * ldx + k0 + ld_c * 8) : zero_u32x4();
      } else {
        stx[i] = ld_global_16(x + (int64_t)row * ldx + k0 + ld_c * 8);
      }
    }
    if constexpr (HAS_W) {
      if constexpr (WDT == kBF16) {
        const uint16_t* wp = reinterpret_cast<const uint16_t*>(w);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          int row = n0 + i * 32 + ld_r;
          row = row < N ? row : N - 1;
          stw[i] = ld_global_16(wp + (int64_t)row * ldw + k0 + ld_c * 8);
        }
      } else {
        // fp8: 64 bytes per row = 4 chunks of 16 fp8; thread handles rows i*64 + tid/4
        const uint8_t* wp = reinterpret_cast<const uint8_t*>(w);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          int row = n0 + i * 64 + (tid >> 2);
          row = row < N ? row : N - 1;
          u32x4_t q = ld_global_16(wp + (int64_t)row * ldw + k0 + (tid & 3) * 16);
          fp8x16_to_bf16x16(q, stw[2 * i], stw[2 * i + 1]);
        }
      }
    }
    if constexpr (IN_T) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        int row = i * 32 + ld_r;
        sta[i] = (row < r) ? ld_global_16(a + (int64_t)row * lda + k0 + ld_c * 8) : zero_u32x4();
      }
    }
  };

  auto store_stage = [&](int stage) {
    char* sx = lds + stage * STAGE_BYTES;
    char* sw = sx + TILE_BYTES;
    char* sa = sw + TILE_BYTES;
#pragma unroll
    for (int i = 0; i < 8; ++i) lds_write16(sx, lds_off(i * 32 + ld_r, ld_c), stx[i]);
    if constexpr (HAS_W) {
      if constexpr (WDT == kBF16) {
#pragma unroll
        for (int i = 0; i < 8; ++i) lds_write16(sw, lds_off(i * 32 + ld_r, ld_c), stw[i]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          int row = i * 64 + (tid >> 2);
          int c = (tid & 3) * 2;
          lds_write16(sw, lds_off(row, c), stw[2 * i]);
          lds_write16(sw, lds_off(row, c + 1), stw[2 * i + 1]);
        }
      }
    }
    if constexpr (IN_T) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        int row = i * 32 + ld_r;
        if (row < rpad32) lds_write16(sa, lds_off(row, ld_c), sta[i]);
      }
    }
  };

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  f32x16_t acct[2][2];  // [rank block][m block] of this wave's 64 T rows
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acct[i][j][v] = 0.f;

  constexpr bool RUN_K = HAS_W || IN_T;
  if constexpr (RUN_K) {
    const int nk = K / BK;
    load_stage(0);
    store_stage(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int stage = kt & 1;
      if (kt + 1 < nk) load_stage((kt + 1) * BK);
      const char* sx = lds + stage * STAGE_BYTES;
      const char* sw = sx + TILE_BYTES;
      const char* sa = sw + TILE_BYTES;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int c = kk * 2 + lh;
        bf16x8_t xf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          xf[j] = as_bf16x8(lds_read16(sx, lds_off(wj * 128 + j * 32 + l32, c)));
        if constexpr (HAS_W) {
          bf16x8_t wf[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            wf[i] = as_bf16x8(lds_read16(sw, lds_off(wi * 128 + i * 32 + l32, c)));
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[i], xf[j], acc[i][j], 0, 0, 0);
        }
        if constexpr (IN_T) {
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) {
            if (rb * 32 < rpad32) {
              bf16x8_t af = as_bf16x8(lds_read16(sa, lds_off(rb * 32 + l32, c)));
#pragma unroll
              for (int jj = 0; jj < 2; ++jj)
                acct[rb][jj] =
                    __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, xf[2 * wi + jj], acct[rb][jj], 0, 0, 0);
            }
          }
        }
      }
      if (kt + 1 < nk) store_stage(stage ^ 1);
      __syncthreads();
    }
  }

  // ---- per-output-channel dequantisation scale (fp8 base) ----
  if constexpr (HAS_W && WDT == kFP8) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          int n = n0 + wi * 128 + i * 32 + g * 8 + lh * 4 + e;
          float sc = w_scale[n < N ? n : N - 1];
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j][g * 4 + e] *= sc;
        }
      }
    }
  }

  // ---- LoRA up-projection: acc[n][m] += sum_j B[n][j] * T[m][j] in 64-rank chunks ----
  if (r > 0) {
    char* st = lds;               // T chunk  [256 m][64 ranks]
    char* sb = lds + TILE_BYTES;  // B chunk  [256 n][64 ranks]
    if constexpr (IN_T) {
      // Park bf16(s * T) for this wave's 64 m rows (m block 2*wi + jj of half wj).
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const int mrow = wj * 128 + (2 * wi + jj) * 32 + l32;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            // ranks rb*32 + 8g + 4*lh + e, e = 0..3  -> 8 contiguous bytes of chunk rb*4+g
            uint32_t lo = pack_bf16x2(s * acct[rb][jj][g * 4 + 0], s * acct[rb][jj][g * 4 + 1]);
            uint32_t hi = pack_bf16x2(s * acct[rb][jj][g * 4 + 2], s * acct[rb][jj][g * 4 + 3]);
            uint2 v;
            v.x = lo;
            v.y = hi;
            *reinterpret_cast<uint2*>(st + lds_off(mrow, rb * 4 + g) + lh * 8) = v;
          }
        }
      }
    }
    const int nrc = (r + 63) / 64;
    for (int rc = 0; rc < nrc; ++rc) {
      const int rk0 = rc * 64;
      // B chunk: rows n0.., ranks rk0 + ld_c*8 (masked beyond r)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int row = n0 + i * 32 + ld_r;
        row = row < N ? row : N - 1;
        int kr = rk0 + ld_c * 8;
        u32x4_t v = (kr < r) ? ld_global_16(bm + (int64_t)row * ldb + kr) : zero_u32x4();
        lds_write16(sb, lds_off(i * 32 + ld_r, ld_c), v);
      }
      if constexpr (!IN_T) {
        // T chunk from the pre-pass workspace (zero-padded to ldt columns)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          int row = m0 + i * 32 + ld_r;
          row = row < M ? row : M - 1;
          lds_write16(st, lds_off(i * 32 + ld_r, ld_c),
                      ld_global_16(tg + (int64_t)row * ldt + rk0 + ld_c * 8));
        }
      }
      __syncthreads();
      const int rem = r - rk0;
      const int nkk = rem >= 64 ? 4 : (rem + 15) / 16;
      for (int kk = 0; kk < nkk; ++kk) {
        const int c = kk * 2 + lh;
        bf16x8_t tf[4], bf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          tf[j] = as_bf16x8(lds_read16(st, lds_off(wj * 128 + j * 32 + l32, c)));
#pragma unroll
        for (int i = 0; i < 4; ++i)
          bf[i] = as_bf16x8(lds_read16(sb, lds_off(wi * 128 + i * 32 + l32, c)));
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[i], tf[j], acc[i][j], 0, 0, 0);
      }
      __syncthreads();
    }
  }

  // ---- store: lane holds y[m][n..n+3] for m = col, n = 8g + 4*lh + (0..3) ----
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + wj * 128 + j * 32 + l32;
    if (m >= M) continue;
    uint16_t* yr = y + (int64_t)m * ldy;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wi * 128 + i * 32 + g * 8 + lh * 4;
        const f32x16_t& c = acc[i][j];
        if (n + 3 < N) {
          uint2 v;
          v.x = pack_bf16x2(c[g * 4 + 0], c[g * 4 + 1]);
          v.y = pack_bf16x2(c[g * 4 + 2], c[g * 4 + 3]);
          *reinterpret_cast<uint2*>(yr + n) = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < N) yr[n + e] = f32_to_bf16_bits(c[g * 4 + e]);
        }
      }
    }
  }
}

// T[m][j] = bf16(s * x[m] . A[j]) for j < r, 0 for r <= j < ldt. One thread per (m, j).
// Pre-pass for ranks above the in-kernel limit.
__global__ void __launch_bounds__(256) down_pad_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                       const uint16_t* __restrict__ a, int64_t lda,
                                                       float s, uint16_t* __restrict__ t,
                                                       int64_t ldt, int64_t M, int64_t K,
                                                       int64_t r) {
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * ldt) return;
  int64_t m = idx / ldt, j = idx % ldt;
  if (j >= r) {
    t[idx] = 0;
    return;
  }
  const u32x4_t* xr = reinterpret_cast<const u32x4_t*>(x + m * ldx);
  const u32x4_t* ar = reinterpret_cast<const u32x4_t*>(a + j * lda);
  float acc = 0.f;
  for (int64_t kc = 0; kc < K / 8; ++kc) {
    u32x4_t xv = xr[kc], av = ar[kc];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc += bf16_bits_to_f32(xv[q] & 0xffffu) * bf16_bits_to_f32(av[q] & 0xffffu);
      acc += bf16_bits_to_f32(xv[q] >> 16) * bf16_bits_to_f32(av[q] >> 16);
    }
  }
  t[idx] = f32_to_bf16_bits(s * acc);
}

template <int WDT, bool HAS_W, bool IN_T, bool GATHER = false>
hipError_t launch_variant(const LoraArgs& p, const uint16_t* tg, int64_t ldt) {
  const int tiles_m = (int)((p.M + BM - 1) / BM);
  const int tiles_n = (int)((p.N + BN - 1) / BN);
  prefill_kernel<WDT, HAS_W, IN_T, GATHER><<<dim3(tiles_m * tiles_n), dim3(NT), 0, p.stream>>>(
      reinterpret_cast<const uint16_t*>(p.x), p.ldx, p.gather, p.gather_rows, p.w, p.ldw, p.w_scale,
      reinterpret_cast<const uint16_t*>(p.a), p.lda, tg, ldt,
      reinterpret_cast<const uint16_t*>(p.b), p.ldb, p.scale,
      reinterpret_cast<uint16_t*>(p.y), p.ldy, (int)p.M, (int)p.N, (int)p.K, (int)p.r, tiles_m);
  return hipGetLastError();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

bool prefill_supported(const LoraArgs& p) {
  if (p.K % BK != 0) return false;
  if (p.M > (int64_t)1 << 30 || p.N > (int64_t)1 << 30 || p.K > (int64_t)1 << 30) return false;
  if (!aligned16(p.x) || p.ldx % 8 != 0) return false;
  if (p.w != nullptr) {
    if (!aligned16(p.w)) return false;
    if (p.w_dtype == kBF16 && p.ldw % 8 != 0) return false;
    if (p.w_dtype == kFP8 && p.ldw % 16 != 0) return false;
  }
  if (p.r > 0) {
    if (p.r % 8 != 0) return false;
    if (!aligned16(p.a) || p.lda % 8 != 0) return false;
    if (!aligned16(p.b) || p.ldb % 8 != 0) return false;
  }
  if ((reinterpret_cast<uintptr_t>(p.y) & 7u) != 0 || p.ldy % 4 != 0) return false;
  return true;
}

size_t prefill_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, int w_dtype) {
  (void)N; (void)K; (void)w_dtype;
  if (r <= RIN) return 0;
  const int64_t ldt = (r + 63) / 64 * 64;
  return (size_t)(M * ldt * 2);
}

hipError_t launch_prefill(const LoraArgs& p) {
  if (p.gather != nullptr) {
    // factorized embedding: gathered x rows, bf16 base, no LoRA term
    return launch_variant<kBF16, true, false, true>(p, nullptr, 0);
  }
  const bool has_w = p.w != nullptr;
  const bool in_t = p.r > 0 && p.r <= RIN;
  const uint16_t* tg = nullptr;
  int64_t ldt = 0;
  if (p.r > RIN) {
    ldt = (p.r + 63) / 64 * 64;
    uint16_t* t = reinterpret_cast<uint16_t*>(p.ws);
    int64_t n = p.M * ldt;
    down_pad_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, p.stream>>>(
        reinterpret_cast<const uint16_t*>(p.x), p.ldx, reinterpret_cast<const uint16_t*>(p.a),
        p.lda, p.scale, t, ldt, p.M, p.K, p.r);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    tg = t;
  }
  if (p.w_dtype == kFP8 && has_w) {
    return in_t ? launch_variant<kFP8, true, true>(p, tg, ldt)
                : launch_variant<kFP8, true, false>(p, tg, ldt);
  }
  if (has_w) {
    return in_t ? launch_variant<kBF16, true, true>(p, tg, ldt)
                : launch_variant<kBF16, true, false>(p, tg, ldt);
  }
  return in_t ? launch_variant<kBF16, false, true>(p, tg, ldt)
              : launch_variant<kBF16, false, false>(p, tg, ldt);
}

}  // namespace wsl
