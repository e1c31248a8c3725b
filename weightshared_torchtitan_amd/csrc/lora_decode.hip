// Decode-shaped (M <= 64 tokens) fused LoRA linear for gfx950.
//
// At small M a projection is a stream over W (N*K elements): the MFMA units are nearly
// idle and the goal is HBM bandwidth, i.e. bytes in flight from the first cycle and as
// few dependent memory round trips and launches as possible. One launch does all of it:
//
//   T workgroups  (blockIdx.x < nT, dispatched first): 16 rows of A each over one K
//                 slice -> T[m][j] = bf16(s * x[m] . A[j]), published to the workspace.
//   W workgroups  (the rest): 16*NR rows of W over one K slice -> base sums, then
//                 y[m][n] = bf16(w_scale[n] * base + T[m] . B[n]).
//
// A workgroup (8 waves) stages its slice of x into LDS with direct global->LDS loads
// (no VGPRs, XOR-swizzled rows), and its B rows likewise, while the first PD K steps of
// its W rows are already in flight into registers. Each lane streams 64 contiguous bytes
// of a row per step (16 rows x 4 lane groups per wave) and v_mfma_f32_16x16x32_bf16
// forms the dot products. The 8 waves form 8/KW row blocks of KW waves each; the KW
// waves of a block interleave over K and their sums are reduced through LDS (KW = 8 for
// K of 8 or more wave steps; short K gives each wave its own rows instead, so a launch
// over a large N and small K, like the tied output head, keeps every wave streaming).
// The up-projection T . B^T of the epilogue is r/32 more MFMAs per 16x16 output block.
//
// Cross-workgroup hand-offs (T to the W workgroups; the partial sums of a K split to
// the last of its workgroups) go through the workspace with agent-scope atomic loads
// and stores, which are coherent across the XCDs' L2s without the whole-L2 write-back
// and invalidate that a device-scope fence costs on this part.
//
// Neither needs a counter: each element is published as one 64-bit word that carries
// the launch's tag (T: bf16 bits under a 48-bit tag with bit 63 set; a partial sum: fp32
// bits under a 31-bit tag, bit 63 clear), so a reader knows an element is this launch's
// by its tag. The tag is the launch ordinal + 1, read from a 64-bit launch counter in
// the workspace prefix: every workgroup adds C / total at exit (workgroup 0 also adds
// C % total), so each launch adds exactly C; a workgroup reads the counter when it
// starts, before its own addition, so floor(count / C) is the ordinal of the running
// launch for every one of its workgroups. Every launch therefore leaves the prefix in a
// valid state without a final barrier. The reader of a K split is its last workgroup.
// Readers wait with a bounded poll on workgroups dispatched before them that never wait
// themselves (T workgroups come first; workgroups are dispatched in index order); past
// the bound a reader computes the missing values itself from x and the weights, so the
// launch always drains.
//
// Optional fusions serve the decode step of the weight-shared Qwen3 harness (bf16 W):
//   RMSNorm prologue   the projection input is bf16(x * rsqrt(mean(x^2) + eps) * w_norm);
//                      the raw rows and w_norm are staged into LDS by direct loads issued
//                      ahead of the W loads, and every workgroup normalises the M rows in
//                      place while its W loads are in flight;
//   SwiGLU epilogue    W holds the gate and up rows interleaved in blocks of 8, so the two
//                      halves of a 16-row MFMA block are g and u of the same 8 outputs, and
//                      y = silu(g) * u;
//   residual epilogue  y = bf16(res + bf16(o)), the block's residual add on the rounded
//                      projection output (y may be res itself).
//
// fp8 base rows are decoded to bf16 in registers (v_cvt_pk_f32_fp8). Reference
// arithmetic: the decode loop runs the same projections at small M
// (scripts/generate/_generation.py:35-80 calling
// torchtitan/models/llama3/model/model.py:189-192,392-398).
#include <algorithm>
#include <climits>
#include <cstring>
#include <cstdlib>
#include <type_traits>

#include "wsl_common.h"

namespace wsl {
namespace {

constexpr int DT = 512;                     // threads per workgroup (8 waves)
constexpr int NWV = DT / 64;
constexpr int64_t LDS_MAX = 160 * 1024;     // gfx950 LDS per workgroup
constexpr int64_t BL_MAX = 32 * 256 * 2;    // B rows of one group: 32 rows x r32 <= 256
constexpr int64_t XS_MAX = LDS_MAX - BL_MAX - 1024;

// The workspace prefix holds the launch counter, spread over kNCnt 64-bit words one
// 128-byte line apart (its value is their sum), so that the exit additions of a launch's
// workgroups do not queue on one address (one word: M = 1, 6144 x 2048 took 11.3 us,
// against 10.2); the rest of the prefix stays zero.
constexpr int kNCnt = 8;
constexpr int kCntStride = 16;  // uint64 words between counters
constexpr uint64_t kLaunchUnit = 1ull << 20;  // C: what one launch adds to the counter
constexpr uint64_t kTagMask = (1ull << 48) - 1;

constexpr int kDefaultSpin = 1 << 16;  // polls of the T counter before computing T locally

// Phase timestamps, in instrumented builds only (-DWSL_STAMPS, libwsl_stamps.so): record
// `bid` slot k gets the 100 MHz constant clock when the workgroup's first thread passes phase
// k. T workgroups: 0 start, 1 partial sums done, 2 T published; W workgroups: 0 start, 1 W
// stream and cross-wave reduction done, 2 K-split reduction done, 3 T gathered, 4 outputs
// stored. Slot 7 holds 1 for a T workgroup, 2 for a W workgroup.
#ifdef WSL_STAMPS
constexpr int kDecStampRecs = 4096;
__device__ unsigned long long g_decode_stamps[kDecStampRecs * 8];
#define WSL_DSTAMP(rec, k)                                                                   \
  do {                                                                                       \
    if (threadIdx.x == 0 && (rec) < kDecStampRecs) g_decode_stamps[(rec) * 8 + (k)] = wall_clock64(); \
  } while (0)
#define WSL_DKIND(rec, v)                                                                    \
  do {                                                                                       \
    if (threadIdx.x == 0 && (rec) < kDecStampRecs) g_decode_stamps[(rec) * 8 + 7] = (v);     \
  } while (0)
#else
#define WSL_DSTAMP(rec, k) \
  do {                     \
  } while (0)
#define WSL_DKIND(rec, v) \
  do {                    \
  } while (0)
#endif
constexpr int LB = 8;                   // workspace loads a thread keeps in flight

typedef __attribute__((address_space(3))) void lds_void_t;

// Cache-policy bits of a direct LDS fill that must see data written in this launch by
// other XCDs (sc1: agent-coherent, as the agent-scope atomic loads use).
constexpr int kAgentCoherent = 16;

// Elements of K one lane covers per step (64 bytes of the row) and per wave step.
template <int WDT> struct Geo {
  static constexpr int LANE_K = (WDT == kFP8) ? 64 : 32;
  static constexpr int WAVE_K = 4 * LANE_K;  // 4 lane groups
};

// s_waitcnt vmcnt(N), expcnt and lgkmcnt unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}

// Workgroup barrier without the fence of __syncthreads() (which would also wait for
// the W loads still in flight); the empty asm keeps LDS accesses on their side.
__device__ __forceinline__ void plain_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// This wave's LDS writes complete (lgkmcnt(0)), then the plain barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);
  plain_barrier();
}

// x slice in LDS: rows 0..M-1, kc bf16 each, 16-byte chunk c of row m stored at chunk
// c ^ (m & 15) (kc is a multiple of 128, so the XOR stays inside the row). The 16 lanes
// that read one chunk index of 16 different rows hit 16 distinct bank groups.
__device__ __forceinline__ int xs_off(int row, int k, int kc) {
  return row * kc * 2 + (((k >> 3) ^ (row & 15)) << 4);
}

// Direct global->LDS fill of x[0..M)[kbeg .. kbeg+kc): the wave instruction j writes
// LDS bytes [1024 j, 1024 j + 1024), lane i the 16 bytes at 1024 j + 16 i. SWZ places the
// chunks as xs_off does; without it the rows are stored as they are.
template <bool SWZ = true, int AUX = 0>
__device__ __forceinline__ void fill_x(char* xs, const uint16_t* __restrict__ x, int64_t ldx,
                                       int M, int kbeg, int kc, int wave, int lane) {
  const int cpr = kc >> 3;  // chunks per row
  const int total = M * cpr;
  for (int j = wave; j * 64 < total; j += NWV) {
    const int p = j * 64 + lane;
    if (p < total) {
      const int row = p / cpr;
      const int c = SWZ ? ((p - row * cpr) ^ (row & 15)) : (p - row * cpr);
      const void* src = x + (int64_t)row * ldx + kbeg + c * 8;
      __builtin_amdgcn_global_load_lds(src, (lds_void_t*)(xs + j * 1024), 16, 0, AUX);
    }
  }
}

// Direct fill of the B rows of a W group: bl[rl][0..r32) for rows row0 + rl (rows past N
// repeat row N-1; chunks past r repeat chunk 0 of the row: finite values that meet the
// zero padding of T).
__device__ __forceinline__ void fill_b(char* bl, const uint16_t* __restrict__ b, int64_t ldb,
                                       int rows, int row0, int nrows, int r, int r32,
                                       int wave, int lane) {
  const int cpr = r32 >> 3;
  const int total = rows * cpr;
  for (int j = wave; j * 64 < total; j += NWV) {
    const int p = j * 64 + lane;
    if (p < total) {
      const int rl = p / cpr;
      int c = p - rl * cpr;
      if (c * 8 >= r) c = 0;
      const int row = min(row0 + rl, nrows - 1);
      const void* src = b + (int64_t)row * ldb + c * 8;
      __builtin_amdgcn_global_load_lds(src, (lds_void_t*)(bl + j * 1024), 16, 0, 0);
    }
  }
}

template <int WDT, int NR>
__device__ __forceinline__ void load_step(u32x4_t (&wv)[NR][4], const void* __restrict__ wmat,
                                          const int64_t (&rowoff)[NR], int kg) {
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if constexpr (WDT == kBF16)
        wv[i][u] = ld_global_16(reinterpret_cast<const uint16_t*>(wmat) + rowoff[i] + kg + u * 8);
      else
        wv[i][u] = ld_global_16(reinterpret_cast<const uint8_t*>(wmat) + rowoff[i] + kg + u * 16);
    }
}

template <int WDT, int NR, int MB>
__device__ __forceinline__ void mma_step(const u32x4_t (&wv)[NR][4], const char* xs, int kc,
                                         const int (&xrow)[MB], int kl, f32x4_t (&acc)[NR][MB]) {
  if constexpr (WDT == kBF16) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      bf16x8_t xf[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        xf[mb] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(xs + xs_off(xrow[mb], kl + u * 8, kc)));
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
          xf[mb] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(xs + xs_off(xrow[mb], kl + u * 16 + h * 8, kc)));
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

struct DecodeArgs {
  const uint16_t* x; int64_t ldx;
  // RMSNorm prologue: x := bf16(x * rsqrt(mean(x^2) + eps) * nw), nw staged at LDS nw_off
  const uint16_t* nw; float eps; int nw_off;
  // residual epilogue: y := bf16(res + bf16(y))
  const uint16_t* res; int64_t ldr;
  const void* w; int64_t ldw; const float* w_scale;
  const uint16_t* a; int64_t lda;
  const uint16_t* b; int64_t ldb;
  uint16_t* y; int64_t ldy;
  float s;
  int M, N, K, r, r32;
  // Grouped launch: T holds rt = groups * r rank columns (A stacked by group); W rows from
  // ge_{g-1} to ge_g belong to group g, whose T columns start at g * r. rt = r and every
  // ge = INT_MAX for a single projection.
  int rt, ge0, ge1, ge2;
  int gT, kst, kct;   // T groups (16 * 8 / KW rows of A), K split and slice
  int gY, ksy, kcy;   // W groups (16*NR rows of W), K split and slice
  int kpt, kpy;       // passes over a T / W slice (x refilled between them)
  int flag_off;       // LDS byte offset of the broadcast word
  unsigned* cnt;      // counter prefix of the workspace
  uint64_t* tfin;     // T [M][rt]: ttag << 16 | bf16 bits
  uint64_t* tpart;    // [gT][kst][T rows per group][M]: ptag << 32 | fp32 partial sum
  uint64_t* ypart;    // [gY][ksy][W rows per group][M]: likewise
  int spin;           // polls of the T counter before the local fallback
  RowMap wmap;        // W and w_scale rows by output row (shared-base forms)
  // greedy-token epilogue (kFuseArgmax): per token m the key am_keys[m * kAmStride] (64-bit
  // atomic max), one arrival counter, the winning index to am_out[m]; LDS scratch at am_red
  uint64_t* am_keys; unsigned* am_cnt; int64_t* am_out; int am_red; int am_total;
};

__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_agent(const unsigned* p) {
  return __hip_atomic_load(const_cast<unsigned*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_agent(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Reads a word and leaves zero in its place (one atomic round trip, like the load).
__device__ __forceinline__ uint64_t take_agent(uint64_t* p) {
  return __hip_atomic_exchange(p, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sums over one K slice of a group of 16*NR rows of `mat` against x (whose fill into
// smem this wave has issued just before), reduced over the waves into sums[row][m]
// (LDS, fp32, stride 16*MB). The x slice's LDS is reused for the reduction.
struct NoPrologue {
  __device__ __forceinline__ void operator()() const {}
};

// Passes over a workgroup's K slice: the slice is walked in `kp` equal parts, and x (rows
// 0..M-1 of `x`) is refilled into the LDS between them, so a slice whose x rows do not fit
// the LDS at once needs no K split across workgroups (and no split hand-off). kp = 1: the
// x slice was filled whole before the call.
struct XPasses {
  const uint16_t* x = nullptr;
  int64_t ldx = 0;
  int kp = 1;
};

// Issued by slice_sums between its first W loads and the wait for the x fill: with
// NoLate the caller has issued the fills before the call; otherwise `late()` issues them
// (after whatever wait it needs), so the W loads are in flight while it waits.
struct NoLate {
  __device__ __forceinline__ void operator()() const {}
};

template <int WDT, int NR, int MB, int KW, class Pro = NoPrologue, class Late = NoLate>
__device__ __forceinline__ void slice_sums(const void* __restrict__ mat, int64_t ldm, int nrows, int row0,
                                           int kbeg, int kc, int M, char* smem, float* sums,
                                           const Pro& pro = Pro(), RowMap rmap = RowMap{},
                                           XPasses xp = XPasses{}, const Late& late = Late()) {
  using G = Geo<WDT>;
  constexpr int PD = NR == 1 ? 4 : (NR == 2 ? 2 : 1);  // K steps in flight per wave (NR*4*PD = 16 loads)
  constexpr int LPS = NR * 4;           // loads per step
  constexpr int MC = 16 * MB;
  constexpr int PER_LANE = NR * MB * 4;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rb = wave / KW, kw = wave % KW;  // row block of this wave, its place along K
  const int l16 = lane & 15;
  const int grp = lane >> 4;
  const int nsteps = kc / G::WAVE_K;
  const int my = nsteps > kw ? (nsteps - kw + KW - 1) / KW : 0;
  const int rbase = row0 + rb * 16 * NR;
  // Passes: each holds kcp columns, kcp / WAVE_K a multiple of KW (the plan's condition), so
  // every wave takes spw steps of each pass and meets the pass barriers with the others.
  const int kcp = kc / xp.kp;
  const int spw = my / xp.kp;

  int64_t rowoff[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) rowoff[i] = (int64_t)map_row(min(rbase + i * 16 + l16, nrows - 1), rmap) * ldm;
  int xrow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) xrow[mb] = min(mb * 16 + l16, M - 1);

  u32x4_t wv[PD][NR][4];
#pragma unroll
  for (int q = 0; q < PD; ++q)
    if (q < my) load_step<WDT, NR>(wv[q], mat, rowoff, kbeg + (kw + q * KW) * G::WAVE_K + grp * G::LANE_K);

  f32x4_t acc[NR][MB];
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[i][mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  if constexpr (std::is_same<Late, NoLate>::value) {
    // The x / B fills were issued before the W loads: wait until only the W loads are
    // outstanding, then for every wave's fills (and LDS writes made before the call).
    const int npf = my < PD ? my : PD;
    if (npf == 0) wait_vm<0>();
    else if (npf == 1) wait_vm<LPS>();
    else if (npf == 2) wait_vm<2 * LPS>();
    else if constexpr (PD == 4) {
      if (npf == 3) wait_vm<3 * LPS>();
      else wait_vm<4 * LPS>();
    }
  } else {
    // The fills follow the W loads: wait for all of them (the W steps, issued first, have
    // had the whole of late()'s wait to land).
    late();
    wait_vm<0>();
  }
  lds_barrier();
  pro();  // the x slice computed from what the fills staged (W loads still in flight)
  if constexpr (!std::is_same<Pro, NoPrologue>::value) plain_barrier();

  int ip = 0, pass = 0;  // step within the pass, pass
  for (int i0 = 0; i0 < my; i0 += PD) {
#pragma unroll
    for (int q = 0; q < PD; ++q) {
      const int i = i0 + q;
      if (i < my) {
        const int kl = (kw + ip * KW) * G::WAVE_K + grp * G::LANE_K;
        mma_step<WDT, NR, MB>(wv[q], smem, kcp, xrow, kl, acc);
        if (i + PD < my)
          load_step<WDT, NR>(wv[q], mat, rowoff, kbeg + (kw + (i + PD) * KW) * G::WAVE_K + grp * G::LANE_K);
        if (++ip == spw && i + 1 < my) {
          // Pass boundary: every wave is done with this pass's x columns; refill them with
          // the next pass's. The fill is younger than the W steps already in flight, so its
          // wait also lands those, which the next MFMAs need first anyway.
          ip = 0;
          ++pass;
          lds_barrier();
          fill_x(smem, xp.x, xp.ldx, M, kbeg + pass * kcp, kcp, wave, lane);
          wait_vm<0>();
          lds_barrier();
        }
      }
    }
  }

  // Cross-wave reduction within each row block (the x slice is dead: its LDS is reused).
  // The first wave of a row block writes its sums in place (D[row][m]: lane holds
  // m = l16, rows grp*4 + e of block i); the others park theirs in `red` in register
  // order, and then every thread finishes a share of the elements, adding the waves in
  // order (a single summing wave was the launch's longest step at 64 rows x 64 tokens).
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
  if (kw > 0) {
    const int slot = rb * (KW - 1) + kw - 1;
#pragma unroll
    for (int i = 0; i < NR; ++i)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          red[(slot * PER_LANE + (i * MB + mb) * 4 + e) * 64 + lane] = acc[i][mb][e];
  } else {
#pragma unroll
    for (int i = 0; i < NR; ++i)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) sums[(rb * 16 * NR + i * 16 + grp * 4 + e) * MC + mb * 16 + l16] = acc[i][mb][e];
  }
  __syncthreads();
  if constexpr (KW > 1) {
    constexpr int EPB = PER_LANE * 64;  // register-order elements of one row block
    for (int gidx = tid; gidx < (NWV / KW) * EPB; gidx += DT) {
      const int rbg = gidx / EPB, el = gidx % EPB;
      const int k = el / 64, ln = el % 64;  // k = (i * MB + mb) * 4 + e
      const int e = k % 4, mb = (k / 4) % MB, i = k / (4 * MB);
      float* dst = sums + (rbg * 16 * NR + i * 16 + (ln >> 4) * 4 + e) * MC + mb * 16 + (ln & 15);
      float v = *dst;
      for (int w2 = 0; w2 < KW - 1; ++w2) v += red[(rbg * (KW - 1) + w2) * EPB + el];
      *dst = v;
    }
    __syncthreads();
  }
}

// One partial sum recomputed from global memory: row `row` of `mat` (bf16 or fp8) against
// x[m] over [kbeg, kbeg + kc). The reducer's fallback past its poll bound.
template <int WDT>
__device__ float direct_partial(const void* __restrict__ mat, int64_t ldm, int row, const uint16_t* __restrict__ x,
                                int64_t ldx, int m, int kbeg, int kc) {
  float acc = 0.f;
  for (int k = kbeg; k < kbeg + kc; ++k) {
    float wv;
    if constexpr (WDT == kFP8)
      wv = __builtin_amdgcn_cvt_pk_f32_fp8((int)reinterpret_cast<const uint8_t*>(mat)[(int64_t)row * ldm + k], false)[0];
    else
      wv = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(mat)[(int64_t)row * ldm + k]);
    acc += wv * bf16_bits_to_f32(x[(int64_t)m * ldx + k]);
  }
  return acc;
}

// The K split of a group. Element q = (row rl, token m), tokens fastest (consecutive
// threads read consecutive LDS words). Every split but the last publishes its partial
// sums as 64-bit words ptag << 32 | fp32 bits (bit 63 clear: never a T word) and is done
// (no wait, no counter). The last split, dispatched after all the others (workgroups are
// dispatched in index order, and the others never wait), polls their words (LB elements
// in flight per thread, one split at a time), sums them in split order with its own last
// (so the result does not depend on timing) and returns true. Past the poll bound it recomputes
// a missing partial from W and x. With one split, returns true at once.
template <int WDT, int ROWS, int MC>
__device__ __forceinline__ bool split_reduce(float* sums, uint64_t* part, int ks, int ksplit, int M, uint32_t ptag,
                                             int spin, const void* mat, int64_t ldm, int nrows, int row0,
                                             const uint16_t* x, int64_t ldx, int kc, RowMap rmap = RowMap{}) {
  if (ksplit == 1) return true;
  const int tid = threadIdx.x;
  const int n = M * ROWS;
  const uint64_t hi = (uint64_t)ptag << 32;
  if (ks < ksplit - 1) {
    for (int q = tid; q < n; q += DT) {
      const int rl = q / M, m = q % M;
      st_agent(part + (int64_t)ks * n + q, hi | __float_as_uint(sums[rl * MC + m]));
    }
    return false;
  }
  // The words of SC splits are requested together (one memory round trip for up to SC
  // splits, where one split at a time cost a round trip each: M = 64, K = 6144 has six
  // splits); they are still added in split order. Each word is taken (exchanged with zero)
  // rather than loaded, so a partial does not outlive its launch: the 31-bit tag repeats
  // after 2^31 - 1 launches, and a word left in a region no later launch rewrote could
  // otherwise match a launch that far ahead. Zero matches no tag; a word taken before its
  // writer stored it is polled again. One exception: when the poll bound runs out the
  // reducer recomputes that split locally (direct_partial), and the late writer's word then
  // lands after the last take and stays in the workspace, tagged with this launch.
  constexpr int SC = 4;
  for (int q0 = 0; q0 < n; q0 += LB * DT) {
    float v[LB];
#pragma unroll
    for (int u = 0; u < LB; ++u) v[u] = 0.f;
    for (int sp0 = 0; sp0 < ksplit - 1; sp0 += SC) {
      const int nsc = min(SC, ksplit - 1 - sp0);
      uint64_t w[SC][LB];
#pragma unroll
      for (int c = 0; c < SC; ++c)
#pragma unroll
        for (int u = 0; u < LB; ++u) {
          const int q = q0 + u * DT + tid;
          w[c][u] = (c < nsc && q < n) ? take_agent(part + (int64_t)(sp0 + c) * n + q) : 0;
        }
#pragma unroll
      for (int c = 0; c < SC; ++c) {
        if (c >= nsc) break;
        const int sp = sp0 + c;
        uint64_t* ps = part + (int64_t)sp * n;
#pragma unroll
        for (int u = 0; u < LB; ++u) {
          const int q = q0 + u * DT + tid;
          if (q < n) {
            for (int it = 0; (w[c][u] >> 32) != ptag && it < spin; ++it) w[c][u] = take_agent(ps + q);
            const int rl = q / M, m = q % M;
            v[u] += (w[c][u] >> 32) == ptag
                        ? __uint_as_float((uint32_t)w[c][u])
                        : direct_partial<WDT>(mat, ldm, map_row(min(row0 + rl, nrows - 1), rmap), x, ldx, m,
                                              sp * kc, kc);
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < LB; ++u) {
      const int q = q0 + u * DT + tid;
      if (q < n) {
        const int rl = q / M, m = q % M;
        sums[rl * MC + m] = v[u] + sums[rl * MC + m];
      }
    }
  }
  __syncthreads();
  return true;
}

// Sum of the kNCnt counter words, which every group of kNCnt consecutive lanes holds once
// (every lane gets the total).
__device__ __forceinline__ uint64_t count_sum(uint64_t v) {
#pragma unroll
  for (int o = kNCnt / 2; o > 0; o >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, o, 64), hi = __shfl_xor((uint32_t)(v >> 32), o, 64);
    v += ((uint64_t)hi << 32) | lo;
  }
  return v;
}

// Tags of the two kinds of hand-off word. A T word's upper 48 bits are 1 << 47 | the low
// 47 bits of the launch tag; a partial-sum word's upper 32 bits are the launch tag folded
// into [1, 2^31 - 1], so bit 63 tells the kinds apart (workspaces are shared by launches
// of different shapes, whose regions overlap) and a zero word matches neither.
__device__ __forceinline__ uint64_t ttag_of(uint64_t tag) { return (1ull << 47) | (tag & ((1ull << 47) - 1)); }
__device__ __forceinline__ uint32_t ptag_of(uint64_t tag) { return (uint32_t)((tag - 1) % 0x7fffffffull) + 1u; }

// T[m][j] (bf16) into LDS tl[m][0..r32) (row stride r32 + 8 elements), zero for m >= M
// or j >= r. Polls (bounded) until every element carries this launch's tag; past the
// bound computes T itself from x and A.
// Eight consecutive elements of the projection input x[m][k..k+8): x itself, or with the
// RMSNorm prologue bf16(x * rsqrt(ss[m] / K + eps) * w_norm).
template <bool NORM, bool COH = false>
__device__ __forceinline__ void load_x8(const DecodeArgs& p, const float* ss, int m, int k, float (&v)[8]) {
  u32x4_t xv;
  if constexpr (COH) {  // x written earlier in this launch (a chain stage), maybe on another XCD
    const uint64_t* q = reinterpret_cast<const uint64_t*>(p.x + (int64_t)m * p.ldx + k);
    const uint64_t lo = ld_agent(q), hi = ld_agent(q + 1);
    xv = u32x4_t{(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)};
  } else {
    xv = ld_global_16(p.x + (int64_t)m * p.ldx + k);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = bf16_bits_to_f32((xv[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
  if constexpr (NORM) {
    const u32x4_t wv = ld_global_16(p.nw + k);
    const float inv = rsqrtf(ss[m] / (float)p.K + p.eps);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      v[e] = bf16_bits_to_f32(f32_to_bf16_bits(v[e] * inv * bf16_bits_to_f32((wv[e >> 1] >> ((e & 1) * 16)) & 0xffffu)));
  }
}

template <int MC, bool NORM = false, bool COH = false>
__device__ __forceinline__ void gather_t(const DecodeArgs& p, uint16_t* tl, uint64_t tag, int* flag,
                                         const float* ss = nullptr, int goff = 0) {
  const int tid = threadIdx.x;
  const int tls = p.r32 + 8;
  const uint64_t ttag = ttag_of(tag);
  for (int q = tid; q < MC * tls; q += DT) tl[q] = 0;
  const int n = p.M * p.r;
  if (tid == 0) *flag = 0;
  __syncthreads();
  // Each thread spins on its own elements (bounded; LB loads in flight per round), so an
  // element is taken as soon as it is visible, without a workgroup round per poll.
  for (int q0 = 0; q0 < n; q0 += LB * DT) {
    uint64_t v[LB];
#pragma unroll
    for (int u = 0; u < LB; ++u) {
      const int q = min(q0 + u * DT + tid, n - 1);
      v[u] = ld_agent(p.tfin + (q / p.r) * p.rt + goff + q % p.r);
    }
#pragma unroll
    for (int u = 0; u < LB; ++u) {
      const int q = q0 + u * DT + tid;
      if (q < n) {
        const int m = q / p.r, j = q % p.r;
        const uint64_t* src = p.tfin + m * p.rt + goff + j;
        for (int it = 0; (v[u] >> 16) != ttag && it < p.spin; ++it) v[u] = ld_agent(src);
        if ((v[u] >> 16) != ttag) *flag = 1;
        tl[m * tls + j] = (uint16_t)(v[u] & 0xffffu);
      }
    }
  }
  __syncthreads();
  const bool ok = *flag == 0;
  __syncthreads();  // every thread has read the flag before anyone reuses it
  if (!ok) {
    for (int q = tid; q < n; q += DT) {
      const int m = q / p.r, j = q % p.r;
      const uint16_t* ar = p.a + (int64_t)(goff + j) * p.lda;
      float acc = 0.f;
      for (int k = 0; k < p.K; k += 8) {
        float xv[8];
        load_x8<NORM, COH>(p, ss, m, k, xv);
        const u32x4_t av = ld_global_16(ar + k);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += xv[e] * bf16_bits_to_f32((av[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
      }
      tl[m * tls + j] = f32_to_bf16_bits(p.s * acc);
    }
  }
  __syncthreads();
}

constexpr int NORM_CH = 4;  // 16-byte chunks of x per thread in the RMSNorm prologue
constexpr int kFuseNorm = 1, kFuseAct = 2, kFuseRes = 4, kFuseArgmax = 8;
constexpr int kAmStride = 32;  // uint64 words between two tokens' keys (256 bytes)
constexpr int kNormLds = 64 * 4 + NORM_CH * DT / 16 * 4;  // row sums + slots

// RMSNorm prologue, run by slice_sums once the direct fills have landed: the raw rows
// x[0..M)[0..K) sit unswizzled in the x-slice region (chunk q of the M*K/8 at byte 16 q)
// and w_norm at nws. Each thread takes up to NORM_CH chunks into registers; every 16
// consecutive chunks (one 16-lane group, inside one row as K/8 is a multiple of 16) leave
// their sum of squares in slot q/16, so row m owns the K/128 slots from m*K/128 on and its
// sum is taken over them in a fixed order (plain LDS stores: an LDS atomic would make the
// compiler wait for the W loads in flight). After a barrier every chunk is written back at
// its swizzled place as bf16(x * rsqrt(sum / K + eps) * w_norm); threads m < M also leave
// the row sum in ss[m] for the T fallback.
struct NormPrologue {
  const DecodeArgs* p;
  char* xs;
  float* ss;      // [64] row sums, then [NORM_CH * DT / 16] slots
  const char* nws;

  __device__ __forceinline__ float row_sum(const float* slots, int m, int spr) const {
    float t = 0.f;
    for (int k = 0; k < spr; ++k) t += slots[m * spr + k];
    return t;
  }

  __device__ __forceinline__ void operator()() const {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int cpr = p->K >> 3;
    const int spr = cpr >> 4;  // slots per row
    const int total = p->M * cpr;
    float* slots = ss + 64;
    float h[NORM_CH][8];
#pragma unroll
    for (int j = 0; j < NORM_CH; ++j) {
      const int q = tid + j * DT;
      float part = 0.f;
      if (q < total) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xs + q * 16);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          h[j][e] = bf16_bits_to_f32((v[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
          part += h[j][e] * h[j][e];
        }
      }
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) part += __shfl_xor(part, o, 64);
      if ((lane & 15) == 0 && q < total) slots[q >> 4] = part;
    }
    lds_barrier();  // every chunk is in registers and every slot written
    if (tid < p->M) ss[tid] = row_sum(slots, tid, spr);
#pragma unroll
    for (int j = 0; j < NORM_CH; ++j) {
      const int q = tid + j * DT;
      if (q < total) {
        const int m = q / cpr, c = q - m * cpr;
        const float inv = rsqrtf(row_sum(slots, m, spr) / (float)p->K + p->eps);
        const u32x4_t wv = *reinterpret_cast<const u32x4_t*>(nws + c * 16);
        u32x4_t ov;
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2)
          ov[q2] = pack_bf16x2(h[j][2 * q2] * inv * bf16_bits_to_f32(wv[q2] & 0xffffu),
                               h[j][2 * q2 + 1] * inv * bf16_bits_to_f32(wv[q2] >> 16));
        *reinterpret_cast<u32x4_t*>(xs + xs_off(m, c * 8, p->K)) = ov;
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // written before the caller's barrier
  }
};

// Greedy-token epilogue of a W workgroup: no output is written. Each token's logits over
// this workgroup's rows are rounded to bf16 (the values the unfused head would store), and
// the best (value, lowest index) key per token goes into a 64-bit atomic max. Once this
// workgroup's maxima are performed (vmcnt) it arrives at the counter; the last workgroup to
// arrive takes every key with an atomic exchange (performed where the maxima were, after
// all of them, and leaving zero behind), writes each token's index and returns the counter
// to zero, so every completed launch leaves the keys and the counter zero. The atomics are
// relaxed: the data passed on are the keys themselves, read by atomics at the same scope,
// so no release or acquire is needed, and each of those (an L2 write-back or invalidate)
// cost about 3 us on the launch (C4 head, 396 workgroups: 27.8 against 30.8 us; the GEMV
// without the epilogue 21.8). Spreading the arrivals over 32 counters and a top counter
// was slower still (one more round trip for the last workgroup).
template <int ROWS, int MC>
__device__ __forceinline__ void argmax_epilogue(const DecodeArgs& p, const float* sums, int row0, char* smem) {
  constexpr int RG = DT / MC;  // row groups
  const int tid = threadIdx.x;
  const int tok = tid % MC, rg = tid / MC;
  uint64_t* red = reinterpret_cast<uint64_t*>(smem + p.am_red);
  int* last = reinterpret_cast<int*>(red + DT);  // dynamic LDS: the kernel takes the full LDS as dynamic
  uint64_t best = 0;
  if (tok < p.M) {
    for (int rl = rg; rl < ROWS; rl += RG) {
      const int n = row0 + rl;
      if (n < p.N) {
        float v = sums[rl * MC + tok];
        if (p.w_scale != nullptr) v *= p.w_scale[map_row(n, p.wmap)];
        const uint64_t k = am_key(bf16_round(v), n);
        best = k > best ? k : best;
      }
    }
  }
  red[rg * MC + tok] = best;
  __syncthreads();
  if (tid < p.M) {
    uint64_t b = 0;
    for (int q = 0; q < RG; ++q) {
      const uint64_t v = red[q * MC + tid];
      b = v > b ? v : b;
    }
    if (b != 0) __hip_atomic_fetch_max(p.am_keys + (size_t)tid * kAmStride, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  wait_vm<0>();     // every maximum of this workgroup is performed
  __syncthreads();  // ... before its arrival
  if (tid == 0) {
    const unsigned old = __hip_atomic_fetch_add(p.am_cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *last = old == (unsigned)(p.am_total - 1);
  }
  __syncthreads();
  if (!*last) return;
  if (tid < p.M) p.am_out[tid] = am_index(take_agent(p.am_keys + (size_t)tid * kAmStride));
  if (tid == 0) __hip_atomic_store(p.am_cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- Chains (wsl_lora_linear_chain_fwd): the stages of one persistent launch ----
// A W workgroup of a chain stage publishes one word per workgroup once its outputs are
// stored (agent-scope stores, then vmcnt(0)); a stage that reads an earlier stage's output
// waits, after issuing its first W loads, until every word of the previous stage carries the
// launch's flag value, and only then fetches x (agent-coherent loads: another XCD wrote it).
// The flag value's top bits (0x7F5A) are neither a T word's (bit 63 set) nor, for the first
// 2^30 launches, a partial-sum word's.
struct ChainCtl {
  const uint64_t* prev_flags;  // W workgroup words of the stage waited on; nullptr: no wait
  int prev_n;
  uint64_t* flags;             // this stage's W workgroup words
  unsigned* err;               // sticky failure word of the launch (a wait that gave up)
  int spin;
};
__device__ __forceinline__ uint64_t chain_flag_of(uint64_t tag) { return (0x7F5Aull << 48) | (tag & kTagMask); }

// Wave 0 polls the previous stage's words (bounded, with a short sleep between rounds), then
// every wave passes a barrier: no x or residual load of this workgroup is issued before the
// previous stage's outputs are out. The barrier carries no fence, so the W loads already in
// flight stay in flight.
__device__ __forceinline__ void chain_wait(const ChainCtl* c, uint64_t tag) {
  if (c->prev_flags == nullptr) return;
  if (threadIdx.x < 64) {
    const uint64_t want = chain_flag_of(tag);
    // up to 8 flags per lane requested together (one round trip for 512 flags), then each
    // one not yet set is polled
    constexpr int FB = 8;
    bool ok = true;
    for (int i0 = 0; i0 < c->prev_n; i0 += 64 * FB) {
      uint64_t v[FB];
#pragma unroll
      for (int u = 0; u < FB; ++u) {
        const int i = i0 + u * 64 + (int)threadIdx.x;
        v[u] = i < c->prev_n ? ld_agent(c->prev_flags + i) : want;
      }
#pragma unroll
      for (int u = 0; u < FB; ++u) {
        const int i = i0 + u * 64 + (int)threadIdx.x;
        for (int it = 0; v[u] != want && it < c->spin; ++it) {
          __builtin_amdgcn_s_sleep(1);
          v[u] = ld_agent(c->prev_flags + i);
        }
        ok = ok && v[u] == want;
      }
    }
    if (!ok) __hip_atomic_fetch_or(c->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  plain_barrier();
}

// Eight bytes of y: a plain store, or in a chain an agent-scope one (read by other XCDs in
// the same launch).
template <bool CH>
__device__ __forceinline__ void store_out8(uint16_t* q, uint2 v) {
  if constexpr (CH)
    st_agent(reinterpret_cast<uint64_t*>(q), ((uint64_t)v.y << 32) | v.x);
  else
    *reinterpret_cast<uint2*>(q) = v;
}

// The work of one workgroup of a decode launch: a T workgroup (bid < gT * kst) or a W
// workgroup. CH: a stage of a chain (ctl), see ChainCtl: its first W (or A) loads are issued
// before it waits for its input.
template <int WDT, int NR, int MB, int KW, int FUSE, bool CH = false>
__device__ __forceinline__ void decode_body(const DecodeArgs& p, int bid, uint64_t cnt_raw, char* smem,
                                            const ChainCtl* ctl = nullptr) {
  constexpr bool NORM = (FUSE & kFuseNorm) != 0;
  constexpr bool ACT = (FUSE & kFuseAct) != 0;
  constexpr bool RES = (FUSE & kFuseRes) != 0;
  constexpr int RBK = NWV / KW;         // row blocks per workgroup
  constexpr int ROWS = RBK * 16 * NR;   // W rows per workgroup
  constexpr int TROWS = RBK * 16;       // A rows per T workgroup
  constexpr int MC = 16 * MB;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nT = p.gT * p.kst;
  int* flag = reinterpret_cast<int*>(smem + p.flag_off);
  // The launch counter was loaded at entry. The tag is formed where it is first needed,
  // behind an empty asm: formed at entry, its wait for the load (a memory round trip)
  // held back every workgroup's first W and x loads.
  const auto late_tag = [cnt_raw]() {
    uint64_t c = cnt_raw;
    asm volatile("" : "+v"(c));
    return (count_sum(c) / kLaunchUnit + 1) & kTagMask;
  };

  if (bid < nT) {
    // ---------------- T workgroup: TROWS rows of A over one K slice
    WSL_DSTAMP(bid, 0);
    WSL_DKIND(bid, 1);
    const int g = bid / p.kst, ks = bid % p.kst;
    const int kbeg = ks * p.kct;
    constexpr int RED_T = (NWV - RBK) * MB * 4 * 64 * 4;
    float* sums = reinterpret_cast<float*>(smem + RED_T);
    if constexpr (CH) {  // one K slice, no passes: A loads first, then the wait, then x
      float* ss = reinterpret_cast<float*>(smem + p.flag_off + 16);
      const auto late = [&]() {
        chain_wait(ctl, late_tag());
        if constexpr (NORM) {
          fill_x<false, kAgentCoherent>(smem, p.x, p.ldx, p.M, 0, p.K, wave, lane);
          fill_x<false>(smem + p.nw_off, p.nw, 0, 1, 0, p.K, wave, lane);
        } else {
          fill_x<true, kAgentCoherent>(smem, p.x, p.ldx, p.M, 0, p.K, wave, lane);
        }
      };
      if constexpr (NORM)
        slice_sums<kBF16, 1, MB, KW>(p.a, p.lda, p.rt, g * TROWS, 0, p.kct, p.M, smem, sums,
                                     NormPrologue{&p, smem, ss, smem + p.nw_off}, RowMap{}, XPasses{}, late);
      else
        slice_sums<kBF16, 1, MB, KW>(p.a, p.lda, p.rt, g * TROWS, 0, p.kct, p.M, smem, sums, NoPrologue{},
                                     RowMap{}, XPasses{}, late);
    } else if constexpr (NORM) {  // one K slice (kst == 1): the whole rows
      float* ss = reinterpret_cast<float*>(smem + p.flag_off + 16);
      fill_x<false>(smem, p.x, p.ldx, p.M, 0, p.K, wave, lane);
      fill_x<false>(smem + p.nw_off, p.nw, 0, 1, 0, p.K, wave, lane);
      slice_sums<kBF16, 1, MB, KW>(p.a, p.lda, p.rt, g * TROWS, kbeg, p.kct, p.M, smem, sums,
                                   NormPrologue{&p, smem, ss, smem + p.nw_off});
    } else {
      fill_x(smem, p.x, p.ldx, p.M, kbeg, p.kct / p.kpt, wave, lane);
      slice_sums<kBF16, 1, MB, KW>(p.a, p.lda, p.rt, g * TROWS, kbeg, p.kct, p.M, smem, sums, NoPrologue{},
                                   RowMap{}, XPasses{p.x, p.ldx, p.kpt});
    }
    WSL_DSTAMP(bid, 1);
    const uint64_t tag = late_tag();
    if (split_reduce<kBF16, TROWS, MC>(sums, p.tpart + (int64_t)g * p.kst * p.M * TROWS, ks, p.kst, p.M,
                                       ptag_of(tag), p.spin, p.a, p.lda, p.rt, g * TROWS, p.x, p.ldx,
                                       p.kct)) {
      for (int q = tid; q < p.M * TROWS; q += DT) {
        const int m = q / TROWS, rl = q % TROWS, j = g * TROWS + rl;
        if (j < p.rt) st_agent(p.tfin + m * p.rt + j, (ttag_of(tag) << 16) | f32_to_bf16_bits(p.s * sums[rl * MC + m]));
      }
      WSL_DSTAMP(bid, 2);
    }
  } else {
    // ---------------- W workgroup: 16*NR rows of W over one K slice
    WSL_DSTAMP(bid, 0);
    WSL_DKIND(bid, 2);
    const int yb = bid - nT;
    const int g = yb / p.ksy, ks = yb % p.ksy;
    const int kbeg = ks * p.kcy;
    const int row0 = g * ROWS;
    constexpr int RED = (NWV - RBK) * NR * MB * 4 * 64 * 4;
    const int xs_bytes = p.M * (p.kcy / p.kpy) * 2;
    const int post = RED + ROWS * MC * 4 + MC * (p.r32 + 8) * 2;
    char* bl = smem + (xs_bytes > post ? xs_bytes : post);
    float* sums = reinterpret_cast<float*>(smem + RED);
    uint16_t* tl = reinterpret_cast<uint16_t*>(smem + RED + ROWS * MC * 4);
    const int l16 = lane & 15, grp = lane >> 4;
    // Residual epilogue: the residual words of this wave's output blocks are loaded here, so
    // their round trip overlaps the W stream instead of following the T gather. Each element
    // is read and later written by this workgroup only, so y may alias res.
    constexpr int EPB = ((ROWS / 16) * MB + NWV - 1) / NWV;  // epilogue blocks per wave
    uint2 rpre[RES ? EPB : 1];
    const auto load_res = [&]() {
#pragma unroll
      for (int t = 0; t < EPB; ++t) {
        const int blk = wave + t * NWV, i = blk / MB, m = blk % MB * 16 + l16;
        const int n0 = row0 + i * 16 + grp * 4;
        rpre[t] = make_uint2(0u, 0u);
        if (blk < (ROWS / 16) * MB && m < p.M && n0 + 3 < p.N) {
          const uint16_t* q = p.res + (int64_t)m * p.ldr + n0;
          if constexpr (CH) {  // written earlier in this launch, maybe on another XCD
            const uint64_t v = ld_agent(reinterpret_cast<const uint64_t*>(q));
            rpre[t] = make_uint2((uint32_t)v, (uint32_t)(v >> 32));
          } else {
            rpre[t] = *reinterpret_cast<const uint2*>(q);
          }
        }
      }
    };
    if constexpr (RES && !CH) load_res();
    if constexpr (CH) {  // one K slice, no passes: W loads first, then the wait, then x, B, res
      float* ss = reinterpret_cast<float*>(smem + p.flag_off + 16);
      const auto late = [&]() {
        chain_wait(ctl, late_tag());
        if constexpr (NORM) {
          fill_x<false, kAgentCoherent>(smem, p.x, p.ldx, p.M, 0, p.K, wave, lane);
          fill_x<false>(smem + p.nw_off, p.nw, 0, 1, 0, p.K, wave, lane);
        } else {
          fill_x<true, kAgentCoherent>(smem, p.x, p.ldx, p.M, 0, p.K, wave, lane);
        }
        if (p.r > 0) fill_b(bl, p.b, p.ldb, ROWS, row0, p.N, p.r, p.r32, wave, lane);
        if constexpr (RES) load_res();
      };
      if constexpr (NORM)
        slice_sums<WDT, NR, MB, KW>(p.w, p.ldw, p.N, row0, 0, p.kcy, p.M, smem, sums,
                                    NormPrologue{&p, smem, ss, smem + p.nw_off}, p.wmap, XPasses{}, late);
      else
        slice_sums<WDT, NR, MB, KW>(p.w, p.ldw, p.N, row0, 0, p.kcy, p.M, smem, sums, NoPrologue{}, p.wmap,
                                    XPasses{}, late);
    } else if constexpr (NORM) {  // one K slice (ksy == 1): the whole rows
      float* ss = reinterpret_cast<float*>(smem + p.flag_off + 16);
      fill_x<false>(smem, p.x, p.ldx, p.M, 0, p.K, wave, lane);
      fill_x<false>(smem + p.nw_off, p.nw, 0, 1, 0, p.K, wave, lane);
      if (p.r > 0) fill_b(bl, p.b, p.ldb, ROWS, row0, p.N, p.r, p.r32, wave, lane);
      slice_sums<WDT, NR, MB, KW>(p.w, p.ldw, p.N, row0, kbeg, p.kcy, p.M, smem, sums,
                                  NormPrologue{&p, smem, ss, smem + p.nw_off}, p.wmap);
    } else {
      fill_x(smem, p.x, p.ldx, p.M, kbeg, p.kcy / p.kpy, wave, lane);
      if (p.r > 0) fill_b(bl, p.b, p.ldb, ROWS, row0, p.N, p.r, p.r32, wave, lane);
      slice_sums<WDT, NR, MB, KW>(p.w, p.ldw, p.N, row0, kbeg, p.kcy, p.M, smem, sums, NoPrologue{}, p.wmap,
                                  XPasses{p.x, p.ldx, p.kpy});
    }
    WSL_DSTAMP(bid, 1);
    const uint64_t tag = late_tag();
    if (split_reduce<WDT, ROWS, MC>(sums, p.ypart + (int64_t)g * p.ksy * p.M * ROWS, ks, p.ksy, p.M,
                                    ptag_of(tag), p.spin, p.w, p.ldw, p.N, row0, p.x, p.ldx, p.kcy, p.wmap)) {
      WSL_DSTAMP(bid, 2);
      if constexpr ((FUSE & kFuseArgmax) != 0) {  // the head's greedy token: no logits written
        argmax_epilogue<ROWS, MC>(p, sums, row0, smem);
        return;
      }
      if (p.r > 0) {
        const int goff = ((row0 >= p.ge0) + (row0 >= p.ge1) + (row0 >= p.ge2)) * p.r;
        gather_t<MC, NORM, CH>(p, tl, tag, flag, reinterpret_cast<const float*>(smem + p.flag_off + 16), goff);
      }
      WSL_DSTAMP(bid, 3);
      // Epilogue: wave blk finishes the 16 x 16 output block (rows i, tokens mb).
      const int tls = p.r32 + 8;
#pragma unroll
      for (int t = 0; t < EPB; ++t) {
        const int blk = wave + t * NWV;
        if (blk >= (ROWS / 16) * MB) break;
        const int i = blk / MB, mb = blk % MB;
        f32x4_t d = {0.f, 0.f, 0.f, 0.f};
        for (int j0 = 0; j0 < p.r; j0 += 32) {
          const u32x4_t bv = *reinterpret_cast<const u32x4_t*>(bl + ((i * 16 + l16) * p.r32 + j0 + grp * 8) * 2);
          const u32x4_t tv = *reinterpret_cast<const u32x4_t*>(tl + (mb * 16 + l16) * tls + j0 + grp * 8);
          d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(bv), as_bf16x8(tv), d, 0, 0, 0);
        }
        // d: lane holds token m = mb*16 + l16, rows i*16 + grp*4 + e
        const int m = mb * 16 + l16;
        const int n0 = row0 + i * 16 + grp * 4;
        if constexpr (ACT) {
          // rows 0-7 of the block are gate rows, 8-15 the up rows of the same 8 outputs:
          // lane l (groups 0, 1) pairs with lane l + 32 (groups 2, 3)
          float o[4], u[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = sums[(i * 16 + grp * 4 + e) * MC + m] + d[e];
#pragma unroll
          for (int e = 0; e < 4; ++e) u[e] = __shfl_xor(o[e], 32, 64);
          const int f0 = (row0 + i * 16) / 2 + grp * 4;
          if (m < p.M && grp < 2 && 2 * f0 < p.N) {
            uint2 pk;
            pk.x = pack_bf16x2(o[0] / (1.f + __expf(-o[0])) * u[0], o[1] / (1.f + __expf(-o[1])) * u[1]);
            pk.y = pack_bf16x2(o[2] / (1.f + __expf(-o[2])) * u[2], o[3] / (1.f + __expf(-o[3])) * u[3]);
            store_out8<CH>(p.y + (int64_t)m * p.ldy + f0, pk);
          }
        } else if (m < p.M) {
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int n = n0 + e;
            float v = sums[(i * 16 + grp * 4 + e) * MC + m];
            if (p.w_scale != nullptr && n < p.N) v *= p.w_scale[map_row(n, p.wmap)];
            o[e] = v + d[e];
          }
          if constexpr (RES) {  // y = bf16(res + bf16(o)); res may be y itself (read first)
            const uint16_t* rr = p.res + (int64_t)m * p.ldr;
            if (n0 + 3 < p.N) {
              const uint2 rv = rpre[t];
              o[0] = bf16_bits_to_f32(rv.x & 0xffffu) + bf16_round(o[0]);
              o[1] = bf16_bits_to_f32(rv.x >> 16) + bf16_round(o[1]);
              o[2] = bf16_bits_to_f32(rv.y & 0xffffu) + bf16_round(o[2]);
              o[3] = bf16_bits_to_f32(rv.y >> 16) + bf16_round(o[3]);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (n0 + e < p.N) o[e] = bf16_bits_to_f32(rr[n0 + e]) + bf16_round(o[e]);
            }
          }
          uint16_t* yr = p.y + (int64_t)m * p.ldy;
          if (n0 + 3 < p.N) {
            uint2 pk;
            pk.x = pack_bf16x2(o[0], o[1]);
            pk.y = pack_bf16x2(o[2], o[3]);
            store_out8<CH>(yr + n0, pk);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n0 + e < p.N) yr[n0 + e] = f32_to_bf16_bits(o[e]);
          }
        }
      }
      if constexpr (CH) {  // every output of this workgroup is out: publish its word
        wait_vm<0>();
        plain_barrier();
        if (tid == 0) st_agent(ctl->flags + g, chain_flag_of(tag));
      }
      WSL_DSTAMP(bid, 4);
    }
  }
}

// This lane's word of the launch counter (lane % kNCnt), read before this workgroup's exit
// addition; the body sums the words where it forms the launch's tag (see the file comment).
__device__ __forceinline__ uint64_t launch_count(const unsigned* cnt) {
  return ld_agent(reinterpret_cast<const uint64_t*>(cnt) + (threadIdx.x % kNCnt) * kCntStride);
}

// Exit: this workgroup's share of the launch's C (the tag was consumed above), added to
// its own counter word.
__device__ __forceinline__ void launch_exit(unsigned* cnt, int total_wgs) {
  if (threadIdx.x == 0) {
    const uint64_t total = (uint64_t)total_wgs;
    const uint64_t share = kLaunchUnit / total + (blockIdx.x == 0 ? kLaunchUnit % total : 0);
    __hip_atomic_fetch_add(reinterpret_cast<uint64_t*>(cnt) + (blockIdx.x % kNCnt) * kCntStride, share,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int WDT, int NR, int MB, int KW, int FUSE>
__global__ void __launch_bounds__(DT) decode_kernel(DecodeArgs p) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  decode_body<WDT, NR, MB, KW, FUSE>(p, blockIdx.x, launch_count(p.cnt), smem);
  launch_exit(p.cnt, p.gT * p.kst + p.gY * p.ksy);
}

// ---- The chain kernel: the stages of wsl_lora_linear_chain_fwd in one persistent launch ----
constexpr int kChainMax = 8;            // WSL_CHAIN_MAX_STAGES
constexpr int kChainFlagWords = 1024;   // W workgroups per stage
constexpr size_t kChainErrOff = 2048;   // sticky failure word in the counter prefix (unused by other launches)

struct ChainStage {
  DecodeArgs a;
  ChainCtl ctl;
  int fuse, nr, nvb;  // fusion, row blocks per wave, workgroups (T then W)
  int rot;            // workgroup v of the stage runs on workgroup (v + rot) mod grid
};
struct ChainArgs {
  ChainStage st[kChainMax];
  int n;
  unsigned* cnt;
};

template <int NR, int FUSE>
__device__ __forceinline__ void chain_vb(const ChainStage& s, int vb, uint64_t cnt_raw, char* smem) {
  decode_body<kBF16, NR, 1, 8, FUSE, true>(s.a, vb, cnt_raw, smem, &s.ctl);
}

// One workgroup per CU walks every stage in order. Stage s's workgroup v runs on workgroup
// (v + rot_s) mod grid, rot_s being where the stage before it ended (rot_0 = 0), so most of a
// stage lands on workgroups the stage before left idle: those issue their first W loads at
// once and wait for the input with them in flight. A stage's T workgroups (v < nT, at most
// the grid) are in its first round; a workgroup only waits on work of earlier stages or of
// T workgroups, which never wait themselves within their stage.
__global__ void __launch_bounds__(DT, 1) chain_kernel(const ChainArgs args) {
  (void)args;
  // The arguments read where they lie in the kernel argument segment (the first argument is
  // at its start): used by name, the compiler copied them to scratch per lane.
  const ChainArgs& c = *(const ChainArgs*)(const void*)__builtin_amdgcn_kernarg_segment_ptr();
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const uint64_t cnt_raw = launch_count(c.cnt);
  const int grid = (int)gridDim.x;
  for (int s = 0; s < c.n; ++s) {
    const ChainStage& st = c.st[s];
    const int key = st.fuse * 4 + st.nr;
    for (int vb = ((int)blockIdx.x - st.rot + grid) % grid; vb < st.nvb; vb += grid) {
      switch (key) {
        case 0 * 4 + 1: chain_vb<1, 0>(st, vb, cnt_raw, smem); break;
        case 0 * 4 + 2: chain_vb<2, 0>(st, vb, cnt_raw, smem); break;
        case kFuseNorm * 4 + 1: chain_vb<1, kFuseNorm>(st, vb, cnt_raw, smem); break;
        case kFuseNorm * 4 + 2: chain_vb<2, kFuseNorm>(st, vb, cnt_raw, smem); break;
        case (kFuseNorm | kFuseAct) * 4 + 1: chain_vb<1, kFuseNorm | kFuseAct>(st, vb, cnt_raw, smem); break;
        case (kFuseNorm | kFuseAct) * 4 + 2: chain_vb<2, kFuseNorm | kFuseAct>(st, vb, cnt_raw, smem); break;
        case kFuseRes * 4 + 1: chain_vb<1, kFuseRes>(st, vb, cnt_raw, smem); break;
        case kFuseRes * 4 + 2: chain_vb<2, kFuseRes>(st, vb, cnt_raw, smem); break;
        default: break;  // the host plans only the pairs above
      }
      lds_barrier();  // the next workgroup's fills reuse the LDS this one read
    }
  }
  launch_exit(c.cnt, gridDim.x);
}
static_assert(sizeof(ChainArgs) <= 4096, "kernel arguments");

int wave_k_of(int wdt) { return wdt == kFP8 ? 256 : 128; }

// Smallest K split whose x slice (M rows) fits the LDS budget, each slice a whole number
// of wave steps; 0 if none.
int fit_split(int64_t M, int64_t K, int wave_k) {
  for (int64_t s = 1; s * wave_k <= K; ++s) {
    if (K % s != 0 || (K / s) % wave_k != 0) continue;
    if (M * (K / s) * 2 <= XS_MAX) return (int)s;
  }
  return 0;
}

struct DecodePlan {
  int mb, nr, kw, rows, trows, r32;
  int gT, kst, kct;
  int gY, ksy, kcy;
  int kpt, kpy;  // passes over a slice (1: the x slice is filled once)
  size_t off_t, off_pt, off_py, total;
  size_t flag_off, smem;
  bool ok;
};

size_t plan_smem(const DecodePlan& pl, int64_t M, size_t* flag_off) {
  // LDS: max(x slice, reduction + sums + T) + B rows, then the broadcast word.
  const size_t xy = (size_t)pl.kcy / pl.kpy, xt = (size_t)pl.kct / pl.kpt;
  const size_t xs = (size_t)M * (xy > xt ? xy : xt) * 2;
  const size_t red = (size_t)(NWV - NWV / pl.kw) * pl.nr * pl.mb * 4 * 64 * 4;
  const size_t post = red + (size_t)pl.rows * 16 * pl.mb * 4 + (size_t)16 * pl.mb * (pl.r32 + 8) * 2;
  *flag_off = (xs > post ? xs : post) + (size_t)pl.rows * pl.r32 * 2;
  return *flag_off + 16;  // the broadcast word (the RMSNorm prologue adds its own after it)
}

// Modelled time of a plan with `nr` row blocks per wave (16 * nr * 8 / KW rows per W
// workgroup), in us: one workgroup per CU (the x slice holds most of the LDS), so the
// grid runs in ceil(workgroups / 256) waves, each costing a fixed latency plus the
// workgroup's bytes (W rows and x slice) at the rate one CU streams them. Constants from
// M = 32 and 64 sweeps over N, K in {1024, 2048, 6144}: 4 us and 40 GB/s per CU.
double plan_cost(const DecodePlan& pl, int64_t M, int64_t N, int nr) {
  const int64_t rows = (int64_t)(NWV / pl.kw) * 16 * nr;
  const int64_t wgs = (int64_t)pl.gT * pl.kst + (N + rows - 1) / rows * pl.ksy;
  const double waves = (double)((wgs + 255) / 256);
  return waves * (4.0 + (double)((rows + M) * pl.kcy * 2) / 40e3);
}

// Which rows-per-group choices a plan may take: every one (plain launches) or those the
// fused kernels are built for (one token block).
enum class Pick { kAll, kFused, kChain };

// WSL_OPT_DECODE_PASSES: -1 keeps K splits, 1 walks every split slice in passes (one
// workgroup per row group), 0 the measured rule of plan_decode (read per call: a benchmark
// or test can switch it).
enum class PassMode { kAuto, kOff, kOn };
PassMode pass_mode() {
  const int64_t v = option(WSL_OPT_DECODE_PASSES);
  return v < 0 ? PassMode::kOff : v > 0 ? PassMode::kOn : PassMode::kAuto;
}

// rt: rank rows of the T work (groups * r for a grouped launch; r when negative).
// min_splits: K splits of the W work to take at least, where the slices keep eight or more
// whole wave steps (more W workgroups for a launch whose rows alone give few).
DecodePlan plan_decode(int64_t M, int64_t N, int64_t K, int64_t r, int wdt, Pick pick = Pick::kAll,
                       int64_t rt = -1, int min_splits = 1) {
  if (rt < 0) rt = r;
  DecodePlan pl{};
  pl.kpt = pl.kpy = 1;
  pl.mb = (int)((M + 15) / 16);
  if (pl.mb < 1) pl.mb = 1;
  pl.nr = pl.mb >= 3 ? 2 : 1;
  pl.r32 = (int)((r + 31) / 32 * 32);
  pl.ksy = fit_split(M, K, wave_k_of(wdt));
  if (pl.ksy > 0 && min_splits > pl.ksy) {
    const int64_t wk = wave_k_of(wdt);
    for (int64_t s = min_splits; s > pl.ksy; --s)
      if (s % pl.ksy == 0 && K % s == 0 && (K / s) % wk == 0 && (K / s) / wk >= 8) {
        pl.ksy = (int)s;
        break;
      }
  }
  pl.kcy = pl.ksy > 0 ? (int)(K / pl.ksy) : 0;
  if (r > 0) {
    pl.kst = fit_split(M, K, wave_k_of(kBF16));
    pl.kct = pl.kst > 0 ? (int)(K / pl.kst) : 0;
  } else {
    pl.kst = 1;
    pl.kct = (int)K;
  }
  // Waves per row block: all 8 along K when the slice has at least 8 wave steps, else
  // the largest power of two not above the step count (more rows per workgroup), raised
  // again while the B rows do not fit the LDS.
  const int steps = pl.kcy > 0 ? pl.kcy / wave_k_of(wdt) : 8;
  pl.kw = 8;
  while (pl.kw > 1 && pl.kw > steps) pl.kw >>= 1;
  // Short K over very many rows (the tied output head): every wave takes 16-row blocks of
  // its own (three at one token block: 384 rows per workgroup, 396 workgroups for 151936
  // rows, within one wave of two per CU; two blocks gave 594, 1.16 waves), so the grid
  // stays a few per CU.
  if (pl.kw <= 2 && pl.mb <= 2 && N >= 32768) {
    pl.kw = 1;
    pl.nr = pl.mb == 1 ? 3 : 2;
  }
  for (;;) {
    pl.rows = (NWV / pl.kw) * 16 * pl.nr;
    pl.trows = (NWV / pl.kw) * 16;
    if (pl.kw == 8 || plan_smem(pl, M, &pl.flag_off) <= (size_t)LDS_MAX) break;
    pl.kw <<= 1;
  }
  pl.gT = r > 0 ? (int)((rt + pl.trows - 1) / pl.trows) : 0;
  // Whole wave steps along K: rows per workgroup (16, 32 or 64) by the modelled time,
  // among the choices whose LDS fits. (At M = 1 and 8, 6144 x 2048 went 13.0 -> 11.3 us;
  // fp8 at M = 16, 12288 x 4096 went 40.7 -> 20.6 us: one wave of workgroups, not three.)
  const bool can_pick = pick == Pick::kAll || (pick != Pick::kAll && pl.mb == 1);
  if (can_pick && pl.kw == 8 && pl.ksy > 0 && pl.kst > 0) {
    double best = plan_cost(pl, M, N, pl.nr);
    const int legacy = pl.nr;
    for (int nr : {1, 2, 4}) {
      if (nr == legacy || (pick == Pick::kChain && nr > 2)) continue;  // chain kernels: one or two blocks
      DecodePlan c = pl;
      c.nr = nr;
      c.rows = 16 * nr;
      size_t fo;
      if (plan_smem(c, M, &fo) > (size_t)LDS_MAX) continue;
      const double cost = plan_cost(pl, M, N, nr);
      if (cost < best) {
        best = cost;
        pl.nr = nr;
      }
    }
    pl.rows = 16 * pl.nr;
    // The pass form: where x does not fit the LDS whole, one workgroup walks its rows' K
    // range in passes (x refilled between them) instead of spreading it over more K splits.
    // That halves (or more) the workgroups, so a grid that needed two waves of one workgroup
    // per CU may need one, and shortens the split hand-off; each pass boundary costs a
    // refill round trip. Measured at M = 64 on the Qwen3-1.7B shapes (grouped launches):
    // two slices as two passes won everywhere (gate|up 41.7 -> 23.8 us, one wave of
    // workgroups instead of two; q|k|v 19.7 -> 16.9; o 15.7 -> 15.0); six slices (down) as
    // three splits of two passes took 22.1 us against 23.9 for six splits, and as six
    // passes 28.8; three slices (down at M = 32) as passes lost (17.3 -> 19.3). So an even
    // slice count takes two passes per split, with the rows per workgroup the model picks.
    const int wk = wave_k_of(wdt);
    const PassMode mode = pass_mode();
    const bool all_passes = mode == PassMode::kOn;
    const bool w_pass = mode != PassMode::kOff && pl.ksy > 1 && (all_passes || pl.ksy % 2 == 0) &&
                        (pl.kcy / wk) % 8 == 0;
    const bool t_pass = pl.kst > 1 && (all_passes || pl.kst % 2 == 0) && (pl.kct / wave_k_of(kBF16)) % 8 == 0;
    if (w_pass && pick == Pick::kAll) {
      DecodePlan c = pl;
      c.kpy = all_passes ? pl.ksy : 2;
      c.ksy = pl.ksy / c.kpy;
      c.kcy = (int)(K / c.ksy);
      if (t_pass) {
        c.kpt = all_passes ? pl.kst : 2;
        c.kst = pl.kst / c.kpt;
        c.kct = (int)(K / c.kst);
      }
      double pass_best = 1e30;
      for (int nr : {1, 2, 4}) {
        DecodePlan d = c;
        d.nr = nr;
        d.rows = 16 * nr;
        size_t fo;
        if (plan_smem(d, M, &fo) > (size_t)LDS_MAX) continue;
        const double cost = plan_cost(d, M, N, nr);
        if (cost < pass_best) {
          pass_best = cost;
          c.nr = nr;
        }
      }
      if (pass_best < 1e30) {
        c.rows = 16 * c.nr;
        pl = c;
      }
    }
  }
  // Five token blocks and more (65 <= M <= kDecodePlainMaxM, plain bf16 launches; kernels
  // are built for five): x is walked in pass slices of 1024 columns, or 512 where 1024 do
  // not fit the LDS: eight or four wave steps, so four waves run along K and two row
  // blocks share a workgroup.
  // 32 rows per workgroup, or 64 where 32 would take more than one wave of workgroups; the
  // slices are then spread over the largest number of K splits that keeps the grid within
  // one wave of workgroups (more workgroups stream faster; passes spare the workgroups a
  // split hand-off), the rest walked as passes. The split count depends on N through the
  // grid, so above 64 tokens a grouped launch may sum a group's rows in another order than
  // the group's single launch (within the bar; below 65 tokens every choice that fixes the
  // order depends on M and K only, and grouped launches match single ones bit for bit).
  if (pick == Pick::kAll && pl.mb > 4) {
    pl.ok = false;
    const int64_t kcp = (M * 1024 * 2 <= XS_MAX && K % 1024 == 0) ? 1024 : 512;
    if (wdt == kBF16 && K % kcp == 0 && M * kcp * 2 <= XS_MAX) {
      const int slices = (int)(K / kcp);
      pl.kw = 4;
      pl.trows = (NWV / pl.kw) * 16;
      pl.gT = r > 0 ? (int)((rt + pl.trows - 1) / pl.trows) : 0;
      pl.nr = 1;
      pl.rows = (NWV / pl.kw) * 16;
      if ((N + pl.rows - 1) / pl.rows + pl.gT > 256) {
        pl.nr = 2;
        pl.rows *= 2;
      }
      const int64_t gy = (N + pl.rows - 1) / pl.rows;
      int splits = 1;
      for (int d = 1; d <= slices; ++d)
        if (slices % d == 0 && (gy + pl.gT) * d <= 256) splits = d;
      pl.ksy = splits;
      pl.kpy = slices / splits;
      pl.kcy = (int)(K / splits);
      if (r > 0) {
        pl.kst = splits;
        pl.kpt = pl.kpy;
        pl.kct = pl.kcy;
      }
      size_t fo;
      pl.ok = plan_smem(pl, M, &fo) <= (size_t)LDS_MAX;
    }
    if (!pl.ok) return pl;
  }
  pl.gY = (int)((N + pl.rows - 1) / pl.rows);
  pl.ok = pl.ksy > 0 && pl.kst > 0 &&
          (uint64_t)pl.gT * pl.kst + (uint64_t)pl.gY * pl.ksy < kLaunchUnit;
  size_t off = kCounterBytes;
  pl.off_t = off;
  off += (size_t)M * rt * 8;
  off = (off + 255) & ~(size_t)255;
  pl.off_pt = off;
  if (pl.kst > 1) off += (size_t)pl.gT * pl.kst * M * pl.trows * 8;
  off = (off + 255) & ~(size_t)255;
  pl.off_py = off;
  if (pl.ksy > 1) off += (size_t)pl.gY * pl.ksy * M * pl.rows * 8;
  pl.total = off;
  pl.smem = plan_smem(pl, M, &pl.flag_off);
  if (pl.smem > (size_t)LDS_MAX) pl.ok = false;
  return pl;
}

// Lets KERN take the full LDS as dynamic shared memory; set once per kernel (a function-
// local static: thread-safe, one per template instantiation).
template <auto KERN>
hipError_t allow_full_lds() {
  static const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(KERN),
                                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_MAX);
  return e;
}

template <int WDT, int NR, int MB, int KW, int FUSE = 0>
hipError_t launch_one(const DecodeArgs& a, int grid, size_t smem, hipStream_t st) {
  const hipError_t e = allow_full_lds<decode_kernel<WDT, NR, MB, KW, FUSE>>();
  if (e != hipSuccess) return e;
  decode_kernel<WDT, NR, MB, KW, FUSE><<<dim3((unsigned)grid), dim3(DT), smem, st>>>(a);
  return hipGetLastError();
}

template <int FUSE>
hipError_t dispatch_fused(const DecodeArgs& a, int mb, int nr, int grid, size_t smem, hipStream_t st) {
  if (nr == 1 && mb == 1) return launch_one<kBF16, 1, 1, 8, FUSE>(a, grid, smem, st);
  if (nr == 2 && mb == 1) return launch_one<kBF16, 2, 1, 8, FUSE>(a, grid, smem, st);
  if (nr == 4 && mb == 1) return launch_one<kBF16, 4, 1, 8, FUSE>(a, grid, smem, st);
  if (nr == 1 && mb == 2) return launch_one<kBF16, 1, 2, 8, FUSE>(a, grid, smem, st);
  if (nr == 2 && mb == 3) return launch_one<kBF16, 2, 3, 8, FUSE>(a, grid, smem, st);
  if (nr == 2 && mb == 4) return launch_one<kBF16, 2, 4, 8, FUSE>(a, grid, smem, st);
  return hipErrorInvalidValue;  // Pick::kFused plans produce only these pairs
}

// Every (rows per group, token blocks) pair a plan can produce maps to its own kernel; any
// other pair is an error, never a kernel sized for a different plan.
template <int WDT, int KW>
hipError_t dispatch_kw(const DecodeArgs& a, int mb, int nr, int grid, size_t smem, hipStream_t st) {
  if constexpr (KW == 1) {  // the tied head at one token block
    if (nr == 3 && mb == 1) return launch_one<WDT, 3, 1, KW>(a, grid, smem, st);
  }
  if (nr == 1) {
    if (mb == 1) return launch_one<WDT, 1, 1, KW>(a, grid, smem, st);
    if (mb == 2) return launch_one<WDT, 1, 2, KW>(a, grid, smem, st);
    if constexpr (KW == 8) {  // rows per workgroup chosen by plan_cost
      if (mb == 3) return launch_one<WDT, 1, 3, KW>(a, grid, smem, st);
      if (mb == 4) return launch_one<WDT, 1, 4, KW>(a, grid, smem, st);
    }
    if constexpr (KW == 4 && WDT == kBF16) {  // 65 <= M <= kDecodePlainMaxM
      if (mb == 5) return launch_one<WDT, 1, 5, KW>(a, grid, smem, st);
    }
    return hipErrorInvalidValue;
  }
  if (nr == 2) {
    if constexpr (KW == 1) {  // two row blocks per wave at one or two token blocks
      if (mb == 1) return launch_one<WDT, 2, 1, KW>(a, grid, smem, st);
      if (mb == 2) return launch_one<WDT, 2, 2, KW>(a, grid, smem, st);
    }
    if constexpr (KW == 8) {
      if (mb == 1) return launch_one<WDT, 2, 1, KW>(a, grid, smem, st);
      if (mb == 2) return launch_one<WDT, 2, 2, KW>(a, grid, smem, st);
    }
    if (mb == 3) return launch_one<WDT, 2, 3, KW>(a, grid, smem, st);
    if (mb == 4) return launch_one<WDT, 2, 4, KW>(a, grid, smem, st);
    if constexpr (KW == 4 && WDT == kBF16) {  // 65 <= M <= kDecodePlainMaxM
      if (mb == 5) return launch_one<WDT, 2, 5, KW>(a, grid, smem, st);
    }
    return hipErrorInvalidValue;
  }
  if constexpr (KW == 8) {
    if (nr == 4) {
      if (mb == 1) return launch_one<WDT, 4, 1, KW>(a, grid, smem, st);
      if (mb == 2) return launch_one<WDT, 4, 2, KW>(a, grid, smem, st);
      if (mb == 3) return launch_one<WDT, 4, 3, KW>(a, grid, smem, st);
      if (mb == 4) return launch_one<WDT, 4, 4, KW>(a, grid, smem, st);
    }
  }
  return hipErrorInvalidValue;
}

template <int WDT>
hipError_t dispatch(const DecodeArgs& a, int mb, int nr, int kw, int grid, size_t smem, hipStream_t st) {
  switch (kw) {
    case 1: return dispatch_kw<WDT, 1>(a, mb, nr, grid, smem, st);
    case 2: return dispatch_kw<WDT, 2>(a, mb, nr, grid, smem, st);
    case 4: return dispatch_kw<WDT, 4>(a, mb, nr, grid, smem, st);
    default: return dispatch_kw<WDT, 8>(a, mb, nr, grid, smem, st);
  }
}

bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

// Poll bound of the hand-off waits; WSL_OPT_DECODE_SPIN_LIMIT overrides it (a test uses -1,
// no polling, to run the local fallback).
int spin_limit() {
  const int64_t v = option(WSL_OPT_DECODE_SPIN_LIMIT);
  if (v == 0) return kDefaultSpin;
  return v < 0 ? 0 : (int)v;
}

}  // namespace

bool decode_supported(const LoraArgs& p) {
  if (p.M < 1 || p.M > kDecodePlainMaxM) return false;
  if (p.M > kDecodeMaxM) {
    if (p.w_dtype != kBF16) return false;  // fp8 base above 64 tokens: the prefill path
    // 65-72 tokens run on the prefill path's split-K form; WSL_OPT_DECODE_WIDE = 1 takes
    // the wide form here instead (side-by-side timing)
    if (option(WSL_OPT_DECODE_WIDE) <= 0) return false;
  }
  if (p.w == nullptr) return false;  // the delta-only form runs on the prefill path
  if (p.N > (int64_t)1 << 30 || p.K > (int64_t)1 << 30) return false;
  const bool fp8 = p.w_dtype == kFP8;
  if (p.K % wave_k_of(p.w_dtype) != 0) return false;
  if (!aligned16(p.x) || p.ldx % 8 != 0) return false;
  if (!aligned16(p.w) || p.ldw % (fp8 ? 16 : 8) != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.y) & 7u) != 0 || p.ldy % 4 != 0) return false;
  if (p.r > 0) {
    if (p.r % 8 != 0) return false;
    if (!aligned16(p.a) || p.lda % 8 != 0) return false;
    if (!aligned16(p.b) || p.ldb % 8 != 0) return false;
  }
  return plan_decode(p.M, p.N, p.K, p.r, p.w_dtype).ok;
}

// K splits of a fused launch's W work: a residual-epilogue launch (no RMSNorm prologue,
// which needs whole rows in one slice) may take WSL_OPT_DECODE_RES_SPLITS.
int fused_min_splits(int fuse) {
  if (!(fuse & kFuseRes) || (fuse & kFuseNorm)) return 1;
  const int64_t v = option(WSL_OPT_DECODE_RES_SPLITS);
  return v > 1 ? (int)v : 1;
}

// Covers the plain and fused launches' plans of the problem (K splits of a residual
// launch included).
size_t decode_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, int w_dtype) {
  const size_t a = plan_decode(M, N, K, r, w_dtype).total;
  const size_t b = plan_decode(M, N, K, r, w_dtype, Pick::kFused).total;
  const size_t c = plan_decode(M, N, K, r, w_dtype, Pick::kFused, -1, fused_min_splits(kFuseRes)).total;
  return std::max(a, std::max(b, c));
}

namespace {
// cnt: the counter prefix; data: where the plan's workspace offsets (which start after a
// kCounterBytes prefix) are based.
DecodeArgs make_args(const LoraArgs& p, const DecodePlan& pl, char* cnt, char* data) {
  DecodeArgs a{};
  a.x = reinterpret_cast<const uint16_t*>(p.x); a.ldx = p.ldx;
  a.w = p.w; a.ldw = p.ldw; a.w_scale = p.w_scale;
  a.a = reinterpret_cast<const uint16_t*>(p.a); a.lda = p.lda;
  a.b = reinterpret_cast<const uint16_t*>(p.b); a.ldb = p.ldb;
  a.y = reinterpret_cast<uint16_t*>(p.y); a.ldy = p.ldy;
  a.s = p.scale;
  a.M = (int)p.M; a.N = (int)p.N; a.K = (int)p.K; a.r = (int)p.r; a.r32 = pl.r32;
  a.rt = (int)(p.r * p.groups);
  a.ge0 = p.groups > 1 ? (int)p.gend[0] : INT_MAX;
  a.ge1 = p.groups > 2 ? (int)p.gend[1] : INT_MAX;
  a.ge2 = p.groups > 3 ? (int)p.gend[2] : INT_MAX;
  a.gT = pl.gT; a.kst = pl.kst; a.kct = pl.kct;
  a.gY = pl.gY; a.ksy = pl.ksy; a.kcy = pl.kcy;
  a.kpt = pl.kpt; a.kpy = pl.kpy;
  a.flag_off = (int)pl.flag_off;
  a.cnt = reinterpret_cast<unsigned*>(cnt);
  a.tfin = reinterpret_cast<uint64_t*>(data + pl.off_t);
  a.tpart = reinterpret_cast<uint64_t*>(data + pl.off_pt);
  a.ypart = reinterpret_cast<uint64_t*>(data + pl.off_py);
  a.spin = spin_limit();
  a.wmap = p.wmap;
  return a;
}
DecodeArgs make_args(const LoraArgs& p, const DecodePlan& pl) {
  char* ws = reinterpret_cast<char*>(p.ws);
  return make_args(p, pl, ws, ws);
}
}  // namespace

// A grouped launch on the decode path: every group boundary on a W workgroup boundary
// (whole row groups of the plan), so each workgroup's rows take one group's T columns.
bool decode_groups_supported(const LoraArgs& p) {
  if (p.groups < 1 || p.groups > kMaxGroups) return false;
  if (p.groups == 1) return true;
  if (p.r == 0) return false;
  const DecodePlan pl = plan_decode(p.M, p.N, p.K, p.r, p.w_dtype, Pick::kAll, p.r * p.groups);
  if (!pl.ok) return false;
  for (int g = 0; g + 1 < p.groups; ++g)
    if (p.gend[g] % pl.rows != 0) return false;
  return true;
}

size_t decode_grouped_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, int groups, int w_dtype) {
  return plan_decode(M, N, K, r, w_dtype, Pick::kAll, r * groups).total;
}

hipError_t launch_decode(const LoraArgs& p) {
  const DecodePlan pl = plan_decode(p.M, p.N, p.K, p.r, p.w_dtype, Pick::kAll, p.r * p.groups);
  const DecodeArgs a = make_args(p, pl);
  const int grid = pl.gT * pl.kst + pl.gY * pl.ksy;
  return p.w_dtype == kFP8 ? dispatch<kFP8>(a, pl.mb, pl.nr, pl.kw, grid, pl.smem, p.stream)
                           : dispatch<kBF16>(a, pl.mb, pl.nr, pl.kw, grid, pl.smem, p.stream);
}

bool decode_fused_supported(const LoraArgs& p, const FusedArgs& f) {
  if (f.fuse < 1 || f.fuse > 7 || ((f.fuse & kFuseAct) && (f.fuse & kFuseRes))) return false;
  if (p.M > kDecodeMaxM || !decode_supported(p) || p.w_dtype != kBF16) return false;
  const DecodePlan pl = plan_decode(p.M, p.N, p.K, p.r, p.w_dtype, Pick::kFused, -1, fused_min_splits(f.fuse));
  if (!pl.ok || pl.kw != 8) return false;
  if (f.fuse & kFuseNorm) {
    // whole rows in one slice, up to NORM_CH chunks per thread, w_norm staged after the plan's LDS
    if (pl.ksy != 1 || (p.r > 0 && pl.kst != 1)) return false;
    if (p.M * (p.K / 8) > (int64_t)NORM_CH * DT) return false;
    if (f.nw == nullptr || !aligned16(f.nw)) return false;
    if (pl.smem + (size_t)kNormLds + (size_t)p.K * 2 > (size_t)LDS_MAX) return false;
  }
  if ((f.fuse & kFuseAct) && p.N % 16 != 0) return false;
  if (f.fuse & kFuseRes) {
    if (f.res == nullptr || (reinterpret_cast<uintptr_t>(f.res) & 7u) != 0 || f.ldr % 4 != 0) return false;
  }
  return true;
}

// The greedy-token head (kFuseArgmax): a bf16 table, no adapter, one K slice, and one of the
// plans a short-K head over many rows takes (K of two wave steps: one or two token blocks
// with every wave on its own rows, three or four with two waves along K).
namespace {
bool argmax_plan_ok(const DecodePlan& pl) {
  if (!pl.ok || pl.ksy != 1 || pl.gT != 0) return false;
  if (pl.kw == 1) return (pl.nr == 3 && pl.mb == 1) || (pl.nr == 2 && pl.mb == 2);
  if (pl.kw == 2) return pl.nr == 2 && (pl.mb == 3 || pl.mb == 4);
  return false;
}
}  // namespace

bool decode_argmax_supported(const LoraArgs& p) {
  if (p.M > kDecodeMaxM || p.r != 0 || p.w_dtype != kBF16 || !decode_supported(p)) return false;
  return argmax_plan_ok(plan_decode(p.M, p.N, p.K, 0, kBF16, Pick::kFused));
}

// One 256-byte slot per token: the 64-bit key at its start; the slot of token 0 also holds
// the arrival counter, at byte 128.
size_t decode_argmax_keys_bytes(int64_t M) { return (size_t)(M > 1 ? M : 1) * 256; }

hipError_t launch_decode_argmax(const LoraArgs& p, void* keys, int64_t* out) {
  const DecodePlan pl = plan_decode(p.M, p.N, p.K, 0, kBF16, Pick::kFused);
  if (!argmax_plan_ok(pl)) return hipErrorInvalidValue;
  DecodeArgs a = make_args(p, pl);
  a.am_keys = reinterpret_cast<uint64_t*>(keys);
  a.am_cnt = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(keys) + 128);
  a.am_out = out;
  a.am_red = (int)((pl.flag_off + 16 + 7) & ~(size_t)7);
  a.am_total = pl.gY;
  const size_t smem = (size_t)a.am_red + (size_t)DT * 8 + 16;
  if (smem > (size_t)LDS_MAX) return hipErrorInvalidValue;
  const int grid = pl.gY;
  if (pl.kw == 1 && pl.nr == 3) return launch_one<kBF16, 3, 1, 1, kFuseArgmax>(a, grid, smem, p.stream);
  if (pl.kw == 1) return launch_one<kBF16, 2, 2, 1, kFuseArgmax>(a, grid, smem, p.stream);
  if (pl.mb == 3) return launch_one<kBF16, 2, 3, 2, kFuseArgmax>(a, grid, smem, p.stream);
  return launch_one<kBF16, 2, 4, 2, kFuseArgmax>(a, grid, smem, p.stream);
}

hipError_t launch_decode_fused(const LoraArgs& p, const FusedArgs& f) {
  const DecodePlan pl = plan_decode(p.M, p.N, p.K, p.r, p.w_dtype, Pick::kFused, -1, fused_min_splits(f.fuse));
  DecodeArgs a = make_args(p, pl);
  a.nw = reinterpret_cast<const uint16_t*>(f.nw); a.eps = f.eps;
  a.nw_off = (int)pl.flag_off + 16 + kNormLds;
  a.res = reinterpret_cast<const uint16_t*>(f.res); a.ldr = f.ldr;
  const size_t smem = pl.smem + ((f.fuse & kFuseNorm) ? (size_t)kNormLds + (size_t)p.K * 2 : 0);
  const int grid = pl.gT * pl.kst + pl.gY * pl.ksy;
  switch (f.fuse) {
    case kFuseNorm: return dispatch_fused<kFuseNorm>(a, pl.mb, pl.nr, grid, smem, p.stream);
    case kFuseNorm | kFuseAct: return dispatch_fused<kFuseNorm | kFuseAct>(a, pl.mb, pl.nr, grid, smem, p.stream);
    case kFuseAct: return dispatch_fused<kFuseAct>(a, pl.mb, pl.nr, grid, smem, p.stream);
    case kFuseRes: return dispatch_fused<kFuseRes>(a, pl.mb, pl.nr, grid, smem, p.stream);
    case kFuseNorm | kFuseRes: return dispatch_fused<kFuseNorm | kFuseRes>(a, pl.mb, pl.nr, grid, smem, p.stream);
    default: return hipErrorInvalidValue;
  }
}

// ---- Chains ----
namespace {
struct ChainPlan {
  DecodePlan pl[kChainMax];
  size_t data[kChainMax];  // byte offset of stage s's plan region base (its plan offsets add to it)
  size_t smem = 0, total = 0;
  int grid = 0;
  bool ok = false;
};

// The stages' plans (the decode path's one-slice plans of one token block), the workspace
// layout (counter prefix, the stages' flag words, then each stage's hand-off region) and
// the LDS. `cus`: CUs of the device (0: the layout only).
ChainPlan plan_chain(int64_t M, int n, const LoraArgs* ps, const FusedArgs* fs, int cus,
                     const int* after_prev = nullptr) {
  ChainPlan c;
  if (n < 1 || n > kChainMax || M < 1 || M > 16) return c;
  size_t off = kCounterBytes + (size_t)kChainMax * kChainFlagWords * 8;
  int max_t = 0;
  for (int s = 0; s < n; ++s) {
    const LoraArgs& p = ps[s];
    const FusedArgs& f = fs[s];
    const int fuse = f.fuse;
    if (fuse != 0 && fuse != kFuseNorm && fuse != (kFuseNorm | kFuseAct) && fuse != kFuseRes) return c;
    if (fuse != 0 && p.groups != 1) return c;
    if (p.w == nullptr || p.w_dtype != kBF16 || p.w_scale != nullptr || p.wmap.P != 0) return c;
    if (p.M != M || p.N % 16 != 0 || !decode_supported(p)) return c;
    const DecodePlan pl = plan_decode(M, p.N, p.K, p.r, kBF16, Pick::kChain, p.r * p.groups);
    if (!pl.ok || pl.kw != 8 || pl.mb != 1 || pl.nr > 2 || pl.ksy != 1 || pl.kpy != 1) return c;
    if (p.r > 0 && (pl.kst != 1 || pl.kpt != 1)) return c;
    if (pl.gY > kChainFlagWords) return c;
    for (int g = 0; g + 1 < p.groups; ++g)
      if (p.gend[g] % pl.rows != 0) return c;
    size_t smem = pl.smem;
    if (fuse & kFuseNorm) {
      if (p.M * (p.K / 8) > (int64_t)NORM_CH * DT || f.nw == nullptr || !aligned16(f.nw)) return c;
      smem += (size_t)kNormLds + (size_t)p.K * 2;
    }
    if (fuse & kFuseRes) {
      if (f.res == nullptr || (reinterpret_cast<uintptr_t>(f.res) & 7u) != 0 || f.ldr % 4 != 0) return c;
    }
    if (smem > (size_t)LDS_MAX) return c;
    c.pl[s] = pl;
    c.smem = std::max(c.smem, smem);
    c.data[s] = off - kCounterBytes;
    off += ((pl.total - kCounterBytes) + 255) & ~(size_t)255;
    max_t = std::max(max_t, pl.gT * pl.kst);
  }
  // Neighbouring stages whose workgroups together exceed the CUs share some workgroups, and
  // those run the later stage's work only after their own earlier work. In a chain of
  // independent stages, a one-block stage (16 rows per workgroup) with such a neighbour takes
  // 32 rows per workgroup if that removes the overlap and fits the LDS (C3, M = 1, two layers
  // per chain: 3000 against 2514 GB/s with one layer and no widening). With dependent stages
  // it does not: a wider first stage has no earlier stage to stream behind (config 4's decode
  // step: 4941 against 5384 tok/s).
  bool independent = true;
  for (int q = 1; q < n; ++q) independent = independent && (after_prev == nullptr || after_prev[q] == 0);
  if (cus > 0) {
    const auto nvb = [&](int q) { return c.pl[q].gT * c.pl[q].kst + c.pl[q].gY * c.pl[q].ksy; };
    for (int q = 0; q < n && independent && after_prev != nullptr; ++q) {
      DecodePlan& pl = c.pl[q];
      const int prev = q > 0 ? nvb(q - 1) : 0, next = q + 1 < n ? nvb(q + 1) : 0;
      if (pl.nr != 1 || (prev + nvb(q) <= cus && next + nvb(q) <= cus)) continue;
      DecodePlan w = pl;
      w.nr = 2;
      w.rows = 32;
      w.gY = (int)((ps[q].N + 31) / 32);
      const int wv = w.gT * w.kst + w.gY * w.ksy;
      size_t fo;
      const size_t sm = plan_smem(w, M, &fo) + ((fs[q].fuse & kFuseNorm) ? (size_t)kNormLds + (size_t)ps[q].K * 2 : 0);
      bool fits = sm <= (size_t)LDS_MAX;
      for (int g = 0; g + 1 < ps[q].groups; ++g) fits = fits && ps[q].gend[g] % 32 == 0;
      if (!fits || prev + wv > cus || next + wv > cus) continue;
      w.smem = plan_smem(w, M, &w.flag_off);
      pl = w;  // the hand-off regions do not depend on the rows per workgroup (one K slice)
      c.smem = std::max(c.smem, sm);
    }
    int mv = 0;
    for (int q = 0; q < n; ++q) mv = std::max(mv, nvb(q));
    c.grid = std::min(cus, mv);
    if (c.grid < max_t) return c;  // every T workgroup in the first round
  }
  c.total = off;
  c.ok = true;
  return c;
}
}  // namespace

bool decode_chain_supported(int64_t M, int n, const LoraArgs* ps, const FusedArgs* fs) {
  return plan_chain(M, n, ps, fs, 0).ok;
}

size_t decode_chain_workspace_bytes(int64_t M, int n, const LoraArgs* ps, const FusedArgs* fs) {
  const ChainPlan c = plan_chain(M, n, ps, fs, 0);
  return c.ok ? c.total : 0;
}

hipError_t launch_decode_chain(int64_t M, int n, const LoraArgs* ps, const FusedArgs* fs, const int* after_prev,
                               void* ws, hipStream_t stream) {
  const ChainPlan c = plan_chain(M, n, ps, fs, device_cus(), after_prev);
  if (!c.ok || c.grid < 1) return hipErrorInvalidValue;
  char* base = reinterpret_cast<char*>(ws);
  uint64_t* flags = reinterpret_cast<uint64_t*>(base + kCounterBytes);
  ChainArgs a{};
  a.n = n;
  a.cnt = reinterpret_cast<unsigned*>(base);
  for (int s = 0; s < n; ++s) {
    const DecodePlan& pl = c.pl[s];
    DecodeArgs d = make_args(ps[s], pl, base, base + c.data[s]);
    d.nw = reinterpret_cast<const uint16_t*>(fs[s].nw);
    d.eps = fs[s].eps;
    d.nw_off = (int)pl.flag_off + 16 + kNormLds;
    d.res = reinterpret_cast<const uint16_t*>(fs[s].res);
    d.ldr = fs[s].ldr;
    ChainStage& st = a.st[s];
    st.a = d;
    st.fuse = fs[s].fuse;
    st.nr = pl.nr;
    st.nvb = pl.gT * pl.kst + pl.gY * pl.ksy;
    st.rot = s > 0 ? (a.st[s - 1].rot + a.st[s - 1].nvb) % c.grid : 0;
    st.ctl.flags = flags + (size_t)s * kChainFlagWords;
    st.ctl.prev_flags = (s > 0 && after_prev[s]) ? flags + (size_t)(s - 1) * kChainFlagWords : nullptr;
    st.ctl.prev_n = s > 0 ? c.pl[s - 1].gY : 0;
    st.ctl.err = reinterpret_cast<unsigned*>(base + kChainErrOff);
    st.ctl.spin = d.spin;
  }
  const hipError_t e = allow_full_lds<chain_kernel>();
  if (e != hipSuccess) return e;
  chain_kernel<<<dim3((unsigned)c.grid), dim3(DT), c.smem, stream>>>(a);
  return hipGetLastError();
}

size_t decode_chain_err_offset() { return kChainErrOff; }

}  // namespace wsl

#ifdef WSL_STAMPS
// Instrumented builds only: copies the first `recs` decode phase-stamp records (8 words
// each) to host memory, then clears them on the device. Returns 0 or a HIP error code.
extern "C" int wsl_decode_stamps(unsigned long long* host, size_t recs) {
  if (recs > (size_t)wsl::kDecStampRecs) recs = wsl::kDecStampRecs;
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpyFromSymbol(host, HIP_SYMBOL(wsl::g_decode_stamps), recs * 8 * sizeof(unsigned long long));
  static unsigned long long zeros[wsl::kDecStampRecs * 8];
  if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(wsl::g_decode_stamps), zeros, sizeof(zeros));
  return (int)e;
}
#endif
