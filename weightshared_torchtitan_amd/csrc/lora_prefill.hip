// Prefill-shaped fused LoRA linear for gfx950 (CDNA4).
//
//   y[M,N] = (x . W^T) * diag(w_scale) + T . B^T,   T = bf16(s * x . A^T)
//
// Tiling. A workgroup of 8 waves (two per SIMD) owns a BM(m) x BN(n) output tile,
// split over its waves as a WNW x WMW grid of wave tiles; a wave tile is a grid of
// v_mfma_f32_32x32x16_bf16 blocks with fp32 accumulators. Four configurations, chosen
// by how evenly the tiles fill the 256 CUs:
//   256 x 256, 128(n) x 64(m) per wave;
//   256(m) x 192(n), 96 x 64 per wave (N = 3072: two full waves of tiles, not 1.5);
//   128 x 256, 64 x 64 per wave — used when 256-row tiles would leave CUs idle;
//   128 x 128, 64 x 32 per wave (two workgroups fit on a CU) — for shapes that even
//   128 x 256 tiles leave half-idle, and for the split-K rank pre-pass.
// (4-wave tiles, one wave per SIMD, measured slower: 128 x 256 with 128 x 64 per wave ran
// 3-8 % behind the 8-wave 64 x 64 tiling, since one wave per SIMD leaves LDS latency
// exposed; 128 x 128 per wave does not fit its rank blocks beside 256 accumulators.)
// K is walked in 64-wide tiles through two LDS buffers filled by
// global_load_lds_dwordx4 (global memory -> LDS without passing through VGPRs; lane i
// of a wave instruction lands at the wave-uniform LDS base + 16*i, so the XOR swizzle of
// the LDS rows is applied by permuting the global source addresses). The barrier sits
// in the middle of each K tile: the fragments of the tile's last k step are read before
// it, so it frees the buffer for the fill of tile k+2, and the first fragments of tile
// k+1 are read while the last MFMAs of tile k run. Fragments are double-buffered in
// registers across k steps. An fp8 base weight is staged through registers, where it
// is decoded to bf16.
//
// LoRA fusion (rank r <= 64). The rank-r down-projection rides on the main loop: the x
// fragments a wave already holds for x . W^T also feed x . A^T, so T is computed once
// per workgroup from the LDS-resident x tile and never touches HBM. After the K loop T
// is scaled by s, rounded to bf16 and parked in LDS, and the up-projection T . B^T
// accumulates into the same accumulator registers as x . W^T; its B slice is filled
// into the idle LDS buffer while the last K tile is multiplied. For r > 64 a pre-pass
// writes T to the workspace and the kernel consumes it the same way; with N = r the
// pre-pass has few tiles, so it splits K over a second grid dimension into fp32 partials
// that a small kernel sums in split order (deterministic), scales and rounds.
//
// The MFMA "A" operand is the W tile (rows n) and "B" the x tile (rows m): each lane
// ends with 4 consecutive n of one m per accumulator group; the tile is staged through
// LDS and written back as whole rows.
//
// Workgroups are dispatched round-robin over the 8 XCDs; the tile order remaps them so
// that each XCD works on a compact group of m x n tiles and its L2 serves the reuse.
//
// Reference arithmetic being fused: torchtitan/models/llama3/model/model.py:189-192
// (LoRAModule.forward), :392-398 (base projection + broadcast_add with g = 1).
#include <algorithm>
#include <atomic>
#include <climits>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "wsl_common.h"

namespace wsl {
namespace {

constexpr int RIN = 64;   // largest rank whose down-projection runs inside the kernel
constexpr int BK = 64;    // K per LDS buffer
constexpr int ROWB = 128; // bytes per LDS row (BK bf16)
constexpr int KK = 4;     // MFMA k steps per K tile
constexpr int N_XCD = 8;
constexpr int GROUP_M = 4;  // row tiles per XCD group (4 against 8 and 16: +0.9 % at config 2 grouped)
constexpr int kShareClasses = KK;  // shared T (SKT): classes of T's k steps, k step c of every K tile

typedef __attribute__((address_space(3))) void lds_void_t;

// Phase timestamps, in instrumented builds only (-DWSL_STAMPS, libwsl_stamps.so): record
// `rec` (workgroup b's tile q of a strip: 4 b + min(q, 3), b counting the splits of a
// split-K launch as blockIdx.x * gridDim.y + blockIdx.y) slot k gets the 100 MHz constant
// clock when the workgroup's first thread passes phase k: 0 tile start, 1 first K tile
// landed, 2 K loop done, 3 LoRA up-projection done (split-K: before the reduction), 4 output
// staged in LDS, 5 stores issued.
#ifdef WSL_STAMPS
constexpr int kStampRecs = 4096;
__device__ unsigned long long g_prefill_stamps[kStampRecs * 8];
#define WSL_STAMP(rec, k)                                                                  \
  do {                                                                                     \
    if (threadIdx.x == 0 && (rec) < kStampRecs) g_prefill_stamps[(rec) * 8 + (k)] = wall_clock64(); \
  } while (0)
#else
#define WSL_STAMP(rec, k) \
  do {                    \
  } while (0)
#endif

template <int BM_, int BN_, int WNW_, int NW_, int NS_ = 2>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_;
  static constexpr int NS = NS_;                      // LDS ring buffers (K tiles in flight + 1)
  static constexpr int NW = NW_, NT = NW_ * 64;     // waves, threads
  static constexpr int WNW = WNW_, WMW = NW_ / WNW_;  // waves along n and m
  static constexpr int TN = BN / WNW, TM = BM / WMW;  // wave tile
  static constexpr int NI = TN / 32, MJ = TM / 32;    // MFMA blocks per wave
  static constexpr int XB = BM * ROWB, WB = BN * ROWB;
  static constexpr int NXI = XB / 1024 / NW;          // direct-fill instructions per wave
  static constexpr int NWI = WB / 1024 / NW;
  static constexpr int NBI = BN * ROWB / 1024 / NW;   // fills of a [BN][64] B slice
  static_assert(NXI >= 1 && NWI >= 1 && NBI >= 1, "tile too small for the direct-fill split");
};

// Byte offset of 16-byte chunk `c` (0..7) of LDS row `row` (128-byte rows). XOR swizzle
// with row bits 1..3: a ds_read_b128 is served 16 lanes (256 bytes, all 64 banks) at a
// time, and the 16 consecutive rows those lanes read at one chunk index then cover all
// 16 bank groups (row parity picks the half of the banks, the XOR the 16-byte slot).
__device__ __forceinline__ int lds_off(int row, int c) { return row * ROWB + ((c ^ ((row >> 1) & 7)) << 4); }

// Chunk a lane fetches in direct fill number `grp`: the fill writes lane i to LDS slot
// i%8 of row R = grp*8 + i/8, which holds global chunk (i%8) ^ ((R >> 1) & 7).
__device__ __forceinline__ int fill_chunk(int lane, int grp) { return (lane & 7) ^ (((grp & 1) << 2) | (lane >> 4)); }

// gfx950 transposing LDS read (ds_read_b64_tr_b16). Within each 16-lane group, lane i gets
// for e = 0..3 element (i % 4) of the 8 bytes addressed by lane 4e + i / 4 of its group (read
// off the hardware with an in-bounds probe). So if lane j of a group addresses row
// kb + j / 4 at column f0 + 4 (j % 4) of a row-major 16-bit matrix, lane i receives rows
// kb .. kb + 3 of column f0 + i: four k values of one row of the transposed matrix.
typedef short v4i16_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_read_tr8(const char* base, int off) {
  const v4i16_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16_t*)(base + off));
  uint2 r;
  r.x = (uint32_t)(uint16_t)v[0] | ((uint32_t)(uint16_t)v[1] << 16);
  r.y = (uint32_t)(uint16_t)v[2] | ((uint32_t)(uint16_t)v[3] << 16);
  return r;
}

__device__ __forceinline__ u32x4_t lds_read16(const char* base, int off) {
  return *reinterpret_cast<const u32x4_t*>(base + off);
}
__device__ __forceinline__ void lds_write16(char* base, int off, u32x4_t v) {
  *reinterpret_cast<u32x4_t*>(base + off) = v;
}

// A 16-byte chunk of the output: a non-temporal store (y is written once and not read by
// the launch; streamed past the caches it leaves the lines the next launch reads in place).
// Builds with -DWSL_TEMPORAL_STORES (libwsl_temporal.so, for side-by-side timing) store it
// through the caches instead.
__device__ __forceinline__ void store_y16(u32x4_t v, u32x4_t* p) {
#ifdef WSL_TEMPORAL_STORES
  *p = v;
#else
  __builtin_nontemporal_store(v, p);
#endif
}

// A lane offset the compiler must treat as computed here: left visible, the loop-invariant
// zero-extension of each 32-bit offset is hoisted into a live 64-bit register pair, and
// every fill then adds it with a 64-bit VALU op instead of using the uniform-base +
// 32-bit-offset form of the load (measured 2-6 % on the K loop, and 8 fewer VGPRs).
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// One wave instruction: 8 LDS rows starting at row grp*8 of `lds_tile` from `src`
// (this lane's 16 source bytes).
__device__ __forceinline__ void direct_fill(char* lds_tile, int grp, const void* src) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)(lds_tile + grp * 1024), 16, 0, 0);
}

// s_waitcnt vmcnt(0) with expcnt/lgkmcnt left unconstrained (gfx9 encoding).
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0f70); }
// s_waitcnt vmcnt(N), N < 64
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}

// Workgroup barrier of the K loop. Its vmcnt wait is explicit, so it must not carry the
// release fence of __syncthreads(), which would also wait for the fill in flight.
// This wave's LDS reads are complete (lgkmcnt(0)) before it, and the empty asm keeps
// the compiler from moving LDS accesses across it.
__device__ __forceinline__ void ring_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt, expcnt unconstrained
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Calls f(std::integral_constant<int, I>{}) for I = B .. E-1: the k steps of a K tile as
// compile-time indices.
template <int B, int E, class F>
__device__ __forceinline__ void for_ct(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    for_ct<B + 1, E>(f);
  }
}

// SPLIT: split-K plain GEMM for the rank pre-pass. Workgroup row blockIdx.y takes the K
// range [blockIdx.y * K, (blockIdx.y + 1) * K) of x and W and writes its fp32 partial
// product to slice blockIdx.y of y (viewed as fp32 [gridDim.y][M][ldy]).
//
// RED: split-K fused LoRA linear with the reduction in the launch. Workgroup row
// blockIdx.y takes the K range [blockIdx.y * K, (blockIdx.y + 1) * K) of x, W and A (K is
// one split's length); every split writes its fp32 base and T partials to red_part in its
// accumulators' own lane order, and the split that arrives last at the tile's counter
// (red_cnt[blockIdx.x], left at zero again) sums all of them in split order and finishes
// the tile (T, the up-projection, the store) as an unsplit launch would. The sum does not
// depend on which split arrives last, so the result is repeatable bit for bit.
//
// TN: plain GEMM over operands stored with the reduction as rows ("token-major"): x'[m][k] is
// x[k * ldx + m] and W'[n][k] is w[k * ldw + n], as the weight gradients' dY and x are (a
// reduction over the tokens). The tiles go into LDS as they lie, [64 k][BM or BN columns]
// (direct fills, 16-byte chunk c of row k at chunk c ^ 4 (k & 3)), and each MFMA fragment is
// two transposing LDS reads (lds_read_tr8). K rows from `grows` (the token count, from this
// split's start) on are read clamped and zeroed in the x' tile after they land. M and N are
// multiples of 8.
//
// PER: persistent strips. Workgroup b owns `tpw` consecutive column tiles of one row block
// (a strip, all in one group) and runs them one after another. T depends only on the row
// block and the group, so the first tile's K loop computes it (as an unsplit launch does),
// parks it in an LDS region of its own, and the strip's later tiles skip the rank MFMAs
// and the A fills and reuse it.
//
// WT: W' alone token-major, W'[n][k] = w[k * ldw + n] (x', A' and B' as they lie, the rank
// work and epilogue unchanged): the input gradient dX = dY . W + s (dY . B) . A of a linear
// whose W [N, K] is read where it lies, K being the reduction of the forward's output
// columns. The W' tile goes into LDS as [64 k][BN] like the TN operands (every K row is
// in range: K % 64 == 0), and its fragments are the same two transposing reads, whose k
// order (16 kk + 8 (lane / 32) + 0..7) is that of x's plain fragments.
//
// SKT: T shared by the column tiles of a row block and group (launches of one wave of tiles,
// every workgroup resident at once). The group's first kShareClasses tiles each compute one
// class of T's k steps (class c: k step c of every K tile), publish the fp32 partial
// (red_part, lane-major words as RED's records) and arrive at the row block's counter
// (red_cnt[2 rbg]); the other tiles of the group do no rank work. Every tile then waits for
// all the classes, sums them in class order (so every tile of the row block holds the same
// T) and goes on as if it had computed T itself. A wait that runs past skt_spin polls
// computes the classes it has not seen from x and A in global memory (the same k steps in
// the same order: the same bits), so the launch ends whatever the residency; the last
// tile to pass (red_cnt[2 rbg + 1]) returns both counters to zero.
template <class C, int WDT, bool HAS_W, int RB, bool EXT_T, bool GATHER, bool SPLIT = false, bool TN = false,
          bool RED = false, bool PER = false, bool WT = false, bool SKT = false>
__global__ void __launch_bounds__(C::NT, 1)
prefill_kernel(const uint16_t* __restrict__ x, int64_t ldx,
               const int64_t* __restrict__ gidx, int64_t grows,
               const void* __restrict__ w, int64_t ldw, const float* __restrict__ w_scale,
               const uint16_t* __restrict__ a_arg, int64_t lda,
               const uint16_t* __restrict__ tg_arg, int64_t ldt,
               const uint16_t* __restrict__ bm, int64_t ldb, float s, float yscale,
               uint16_t* __restrict__ y, int64_t ldy,
               int M, int N, int K, int r, int tiles_m, int tiles_n,
               int ge0, int ge1, int ge2, int64_t a_gstride, int t_gstride, RowMap wmap,
               uint64_t* __restrict__ red_part, unsigned* __restrict__ red_cnt, int tpw, int skt_spin) {
  constexpr bool W8 = HAS_W && WDT == kFP8;
  constexpr bool WDIRECT = HAS_W && WDT == kBF16;
  constexpr bool LORA = RB > 0 || EXT_T;
  constexpr int NT = C::NT;
  constexpr int AB = RB * 32 * ROWB;         // rank-A slice of a K tile
  constexpr int STAGE = C::XB + C::WB + AB;  // one of the two ring buffers
  constexpr int OS = C::BN * 2 + 16;          // LDS row stride of the staged output tile
  // PER: T of the strip's row block, [BM m][r ranks] bf16, past the ring (rows of 64 bytes
  // for r <= 32, 128 for r <= 64); the staged output tile stays within the ring
  constexpr int TROW = (PER && RB == 1) ? 64 : ROWB;
  constexpr int TREG = PER ? C::BM * TROW : 0;
  constexpr int RING = C::NS * STAGE + TREG;
  constexpr int LDS_BYTES = (RING > C::BM * OS) ? RING : C::BM * OS;
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
  static_assert(!PER || C::BM * OS <= C::NS * STAGE, "staged output clear of the T region");
  static_assert(!PER || (WDT == kBF16 && HAS_W && RB > 0 && !EXT_T && !GATHER && !SPLIT && !TN && !RED && C::NS == 2),
                "persistent strips: bf16 W, in-kernel T, two-buffer ring");
  static_assert(C::BM * ROWB <= STAGE && C::BN * ROWB <= STAGE, "LoRA phase fits the ring");
  __shared__ __attribute__((aligned(1024))) char lds[LDS_BYTES];
  static_assert(!SPLIT || (WDT == kBF16 && HAS_W && RB == 0 && !EXT_T && !GATHER), "split-K is a plain bf16 GEMM");
  static_assert(!TN || (WDT == kBF16 && HAS_W && RB == 0 && !EXT_T && !GATHER), "token-major operands: plain bf16 GEMM");
  static_assert(!RED || (WDT == kBF16 && HAS_W && !EXT_T && !GATHER && !SPLIT && !TN), "in-launch split-K: bf16 W");
  static_assert(C::NS == 2 || (!W8 && !TN && !GATHER), "deep ring: bf16 W and x as they lie");
  static_assert(!WT || (HAS_W && !TN && !GATHER && !SPLIT && !RED && C::BN % 128 == 0 &&
                        (WDT == kBF16 || (C::NS == 2 && (64 * C::BN / 16) % C::NT == 0))),
                "token-major W': x as it lies, 128-column multiples (fp8: two-buffer ring)");
  static_assert(!SKT || (WDT == kBF16 && HAS_W && RB == 1 && !EXT_T && !GATHER && !SPLIT && !TN && !RED && !PER && !WT),
                "shared T: one in-loop rank block, bf16 W, one tile per workgroup");
  int64_t tok_rem = grows;  // TN: K rows from this workgroup's first one to the end (>= 1)
  if constexpr (RED) {
    const int64_t kofs = (int64_t)blockIdx.y * K;
    x += kofs;
    w = reinterpret_cast<const uint16_t*>(w) + kofs;
    if constexpr (RB > 0) a_arg += kofs;
  }
  if constexpr (SPLIT) {
    const int64_t kofs = (int64_t)blockIdx.y * K;
    if constexpr (TN) {
      x += kofs * ldx;
      w = reinterpret_cast<const uint16_t*>(w) + kofs * ldw;
      tok_rem = grows - kofs;
    } else {
      x += kofs;
      w = reinterpret_cast<const uint16_t*>(w) + kofs;
    }
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave index as a scalar: the LDS bases of the direct fills (M0) derive from it
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % C::WNW;
  const int wm = wave / C::WNW;
  const int l32 = lane & 31;
  const int lh = lane >> 5;

  // Byte offset of 16-byte chunk c of row `row` in the T region: 64-byte rows with the
  // chunk XORed by row bits 2..3 (16 consecutive rows at one chunk cover all 64 banks), or
  // the ring's own 128-byte layout.
  auto t_off = [](int row, int c) {
    if constexpr (TROW == 64) return row * 64 + ((c ^ ((row >> 2) & 3)) << 4);
    else return lds_off(row, c);
  };

  // One output tile: tile tq of this workgroup's strip (always 0 without PER). `first`
  // (a compile-time bool) is whether it is the strip's first tile, which computes T.
  auto do_tile = [&](const int tq, auto first) {
  // ---- XCD-aware, grouped tile order (over strips of tpw column tiles with PER) ----
  const int SW = PER ? tpw : 1;
  const int G = tiles_m * tiles_n / SW;
  int t = blockIdx.x;
  if constexpr (PER) asm volatile("" : "+s"(t));  // recomputed per tile, not kept live across tiles
  if (G % N_XCD == 0) t = (t % N_XCD) * (G / N_XCD) + t / N_XCD;
  const int group_size = GROUP_M * (tiles_n / SW);
  const int first_m = (t / group_size) * GROUP_M;
  const int gm = min(tiles_m - first_m, GROUP_M);
  const int tm = first_m + (t % group_size) % gm;
  const int tn = ((t % group_size) / gm) * SW + tq;
  const int m0 = tm * C::BM;
  const int n0 = tn * C::BN;
  // phase-stamp record (split-K launches: one per tile and split)
  const int srec = ((int)blockIdx.x * (int)gridDim.y + (int)blockIdx.y) * 4 + (tq < 3 ? tq : 3);
  (void)srec;
  WSL_STAMP(srec, 0);
  // whether this tile computes T in its K loop (every tile but a strip's later ones)
  constexpr bool t_here = !PER || decltype(first)::value;
  // Grouped launch: output columns [ge_{g-1}, ge_g) are projection g, whose LoRA down
  // factor is rank block g of a (rows g*r..g*r+r-1) and whose T is column block g of the
  // pre-pass output. Group ends are multiples of BN (of a strip's width with PER), so a
  // tile lies in one group; B rows and W rows are indexed by the output column as in a
  // single projection.
  const int grp = (n0 >= ge0) + (n0 >= ge1) + (n0 >= ge2);
  const uint16_t* const a = a_arg + grp * a_gstride;
  const uint16_t* const tg = tg_arg + grp * t_gstride;
  // SKT: the tile's row block and group (rbg), the group's tile count and the tile's class
  // of T's k steps (its column index in the group; -1 past the classes: no rank work)
  int skt_cls = -1, skt_rbg = 0, skt_ntiles = 1;
  if constexpr (SKT) {
    const int gstart = grp == 0 ? 0 : grp == 1 ? ge0 : grp == 2 ? ge1 : ge2;
    const int gend = grp == 0 ? ge0 : grp == 1 ? ge1 : grp == 2 ? ge2 : INT_MAX;
    skt_ntiles = ((gend < N ? gend : N) - gstart + C::BN - 1) / C::BN;
    const int ngroups = 1 + (ge0 != INT_MAX) + (ge1 != INT_MAX) + (ge2 != INT_MAX);
    skt_rbg = tm * ngroups + grp;
    const int local = (n0 - gstart) / C::BN;
    skt_cls = local < kShareClasses ? local : -1;
  }

  // ---- sources of this wave's direct fills: uniform tile base + 32-bit lane offset ----
  const char* xbase = reinterpret_cast<const char*>(GATHER ? x : x + (int64_t)m0 * ldx);
  uint32_t xoff[C::NXI];
  const uint16_t* xg[GATHER ? C::NXI : 1];  // gathered rows keep 64-bit row pointers
#pragma unroll
  for (int i = 0; i < C::NXI; ++i) {
    const int row = (wave * C::NXI + i) * 8 + (lane >> 3);
    const int gr = min(m0 + row, M - 1);
    if constexpr (GATHER) {
      const int64_t id = gidx[gr];
      xg[i] = x + ((id >= 0 && id < grows) ? id : 0) * ldx + fill_chunk(lane, wave * C::NXI + i) * 8;  // bad ids: zeroed at the store
      xoff[i] = 0;
    } else {
      xoff[i] = (uint32_t)((gr - m0) * ldx * 2 + fill_chunk(lane, wave * C::NXI + i) * 16);
    }
  }
  // W rows by output column (mapped for the shared-base forms, whose W is small enough for
  // 32-bit offsets from its start)
  const int wrow0 = wmap.P == 0 ? n0 : 0;
  const char* wbase = reinterpret_cast<const char*>(w) + (WDIRECT ? (int64_t)wrow0 * ldw * 2 : 0);
  uint32_t woff[C::NWI];
#pragma unroll
  for (int i = 0; i < C::NWI; ++i) {
    const int row = (wave * C::NWI + i) * 8 + (lane >> 3);
    woff[i] = (uint32_t)((map_row(min(n0 + row, N - 1), wmap) - wrow0) * ldw * 2 + fill_chunk(lane, wave * C::NWI + i) * 16);
  }
  // WT: the W' tile's direct fills, [64 k][BN] as the TN operands lie: fill q of this wave
  // writes lane i's 16 bytes at 1024 q + 16 i of the tile, row (1024 q + 16 i) / (2 BN), and
  // takes W's column chunk held there (chunk c at physical chunk c ^ 4 (row & 3); columns
  // past N read the last full chunk, their outputs are not stored). The byte offset within
  // a K tile's 64 rows fits 32 bits; the K tile's base is uniform.
  constexpr int QWT = WT ? 64 * C::BN * 2 / 1024 / C::NW : 1;
  uint32_t wtoff[QWT];
  if constexpr (WT && !W8) {
#pragma unroll
    for (int i = 0; i < QWT; ++i) {
      const int q = wave * QWT + i;
      const int row = (q * 1024 + lane * 16) / (C::BN * 2);
      const int c = (lane % (C::BN / 8)) ^ ((row & 3) << 2);
      const int f = min(n0 + c * 8, N - 8);
      wtoff[i] = (uint32_t)(((int64_t)row * ldw + f) * 2);
    }
  }
  // rank-A slice: RB*32 rows = RB*4 fills, one per wave for waves < RB*4 (rows >= r read
  // row r-1; their T ranks are zeroed when T is parked)
  constexpr int NAI = RB * 4;
  uint32_t aoff = 0;
  if constexpr (RB > 0) aoff = (uint32_t)(min(wave * 8 + (lane >> 3), r - 1) * lda * 2 + fill_chunk(lane, wave) * 16);
  // fp8 W: BN rows x 64 B per K tile, 16 fp8 per chunk
  constexpr int W8C = (W8 && !WT) ? C::BN * 4 / NT : 1;  // chunks per thread
  const uint8_t* w8row[W8C];
  if constexpr (W8 && !WT) {
#pragma unroll
    for (int i = 0; i < W8C; ++i) {
      const int id = i * NT + tid;
      w8row[i] = reinterpret_cast<const uint8_t*>(w) + (int64_t)map_row(min(n0 + (id >> 2), N - 1), wmap) * ldw + (id & 3) * 16;
    }
  }

  // TN fills: wave fill q covers LDS bytes [1024 q, 1024 q + 1024) of a [64][cols] tile, lane i
  // the 16 bytes at 1024 q + 16 i: row (1024 q + 16 i) / (2 cols), physical chunk s, which
  // holds column chunk s ^ 4 (row & 3) (clamped to the last full chunk: dropped rows of y)
  auto tn_fill = [&](char* tile, int cols, int q, const uint16_t* src, int64_t ld, int col0, int ncols, int k0) {
    const int cpr = cols / 8;  // 16-byte chunks per row
    const int row = (q * 1024 + lane * 16) / (cols * 2);
    const int sc = lane % cpr;
    const int c = sc ^ ((row & 3) << 2);
    const int f = min(col0 + c * 8, ncols - 8);
    const int64_t t = min((int64_t)(k0 + row), tok_rem - 1);
    direct_fill(tile, q, src + t * ld + f);
  };
  auto issue = [&](int stage, int k0) {
    char* sx = lds + stage * STAGE;
    char* sw = sx + C::XB;
    char* sa = sw + C::WB;
    if constexpr (TN) {
      constexpr int QX = 64 * C::BM * 2 / 1024 / C::NW, QW = 64 * C::BN * 2 / 1024 / C::NW;
#pragma unroll
      for (int i = 0; i < QX; ++i) tn_fill(sx, C::BM, wave * QX + i, x, ldx, m0, M, k0);
#pragma unroll
      for (int i = 0; i < QW; ++i)
        tn_fill(sw, C::BN, wave * QW + i, reinterpret_cast<const uint16_t*>(w), ldw, n0, N, k0);
      return;
    }
#pragma unroll
    for (int i = 0; i < C::NXI; ++i) {
      if constexpr (GATHER) direct_fill(sx, wave * C::NXI + i, xg[i] + k0);
      else direct_fill(sx, wave * C::NXI + i, xbase + k0 * 2 + opaque(xoff[i]));
    }
    if constexpr (WT && !W8) {
      const char* wk = reinterpret_cast<const char*>(w) + (int64_t)k0 * ldw * 2;  // K rows k0..k0+63
#pragma unroll
      for (int i = 0; i < QWT; ++i) direct_fill(sw, wave * QWT + i, wk + opaque(wtoff[i]));
    } else if constexpr (WDIRECT) {
#pragma unroll
      for (int i = 0; i < C::NWI; ++i) direct_fill(sw, wave * C::NWI + i, wbase + k0 * 2 + opaque(woff[i]));
    }
    if constexpr (RB > 0) {
      if (t_here && wave < NAI && (!SKT || skt_cls >= 0))
        direct_fill(sa, wave, reinterpret_cast<const char*>(a) + k0 * 2 + opaque(aoff));
    }
  };
  // B slice [BN][64 ranks from rk0] into `dst`. Lanes past rank r read a finite element
  // of their own row instead; T is zero at those ranks, so they contribute nothing.
  auto issue_b = [&](char* dst, int rk0) {
#pragma unroll
    for (int i = 0; i < C::NBI; ++i) {
      const int grp = wave * C::NBI + i;
      const int row = grp * 8 + (lane >> 3);
      const int kr = rk0 + fill_chunk(lane, grp) * 8;
      const uint16_t* src = bm + (int64_t)min(n0 + row, N - 1) * ldb + (kr < r ? kr : 0);
      direct_fill(dst, grp, src);
    }
  };

  u32x4_t w8stage[W8C];
  // WT with an fp8 W: 64 K rows x BN columns of e4m3 bytes per K tile, 16-byte chunks
  // (row id / (BN / 16), column chunk id % (BN / 16)); each row's scale is that of its
  // reduction index (the linear's output channel), applied as it is decoded
  constexpr int W8T = (W8 && WT) ? 64 * C::BN / 16 / NT : 1;  // chunks per thread
  u32x4_t w8t[W8T];
  float w8s[W8T];
  auto load_w8 = [&](int k0) {
    if constexpr (W8 && WT) {
#pragma unroll
      for (int i = 0; i < W8T; ++i) {
        const int id = i * NT + tid, row = id / (C::BN / 16), c16 = id % (C::BN / 16);
        const int col = min(n0 + c16 * 16, N - 16);  // N % 16 == 0: columns past N read a valid chunk
        w8t[i] = ld_global_16(reinterpret_cast<const uint8_t*>(w) + (int64_t)(k0 + row) * ldw + col);
        w8s[i] = w_scale[k0 + row];
      }
    } else if constexpr (W8) {
#pragma unroll
      for (int i = 0; i < W8C; ++i) w8stage[i] = ld_global_16(w8row[i] + k0);
    }
  };
  // TN: K rows past the token count (clamped reads) are zeroed in the x' tile once it has
  // landed, so they add nothing whatever the W' tile holds there. A thread zeroes chunks
  // that other waves' fills write, and each wave has only waited for its own fills: the
  // barrier first lets every fill land, or a late fill would overwrite the zeros with the
  // clamped row (the weight gradients of a partial token tile then came out wrong now and
  // then).
  auto tn_zero = [&](int stage, int k0) {
    if constexpr (TN) {
      const int64_t valid = tok_rem - k0;
      if (valid < 64) {  // the same for every wave
        ring_barrier();
        char* sx = lds + stage * STAGE;
        const int v0 = valid > 0 ? (int)valid : 0;
        constexpr int CPR = C::BM / 8;
        for (int q = v0 * CPR + tid; q < 64 * CPR; q += NT) lds_write16(sx, q * 16, zero_u32x4());
      }
    }
  };
  auto store_w8 = [&](int stage) {
    if constexpr (W8 && WT) {
      // bf16(code * scale) of each element, into the token-major tile's swizzled chunks
      char* sw = lds + stage * STAGE + C::XB;
#pragma unroll
      for (int i = 0; i < W8T; ++i) {
        const int id = i * NT + tid, row = id / (C::BN / 16), c16 = id % (C::BN / 16);
        const float sc = w8s[i];
        uint32_t o[8];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const auto lo2 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w8t[i][d], false);
          const auto hi2 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w8t[i][d], true);
          o[2 * d] = pack_bf16x2(lo2[0] * sc, lo2[1] * sc);
          o[2 * d + 1] = pack_bf16x2(hi2[0] * sc, hi2[1] * sc);
        }
        const int sw4 = (row & 3) << 2;
        lds_write16(sw, row * C::BN * 2 + (((c16 * 2) ^ sw4) << 4), u32x4_t{o[0], o[1], o[2], o[3]});
        lds_write16(sw, row * C::BN * 2 + (((c16 * 2 + 1) ^ sw4) << 4), u32x4_t{o[4], o[5], o[6], o[7]});
      }
    } else if constexpr (W8) {
      char* sw = lds + stage * STAGE + C::XB;
#pragma unroll
      for (int i = 0; i < W8C; ++i) {
        const int id = i * NT + tid;
        const int row = id >> 2, c = (id & 3) * 2;
        u32x4_t lo, hi;
        fp8x16_to_bf16x16(w8stage[i], lo, hi);
        lds_write16(sw, lds_off(row, c), lo);
        lds_write16(sw, lds_off(row, c + 1), hi);
      }
    }
  };

  // ---- T work split: TBLK (m block, rank block) pairs per wave row (WNW waves) ----
  // With at least WNW blocks every wave takes TPW of them. With fewer (the 128 x 256 tile),
  // one group of TBLK waves per row takes one block each over every k step; successive
  // rows use different groups, so the T waves fall on different SIMDs (wave w runs on
  // SIMD w % 4) and each SIMD carries the same MFMA count.
  constexpr int TBLK = C::MJ * RB;
  constexpr bool ALL_T = RB > 0 && TBLK >= C::WNW;
  constexpr int TPW = (RB == 0) ? 0 : (ALL_T ? TBLK / C::WNW : 1);  // blocks per T wave
  constexpr int TBLKX = TBLK > 0 ? TBLK : 1;  // RB == 0: no T blocks (keeps % and / defined)
  constexpr int TG = (RB == 0 || ALL_T) ? 1 : C::WNW / TBLKX;       // wave groups per row
  static_assert(RB == 0 || TBLK % C::WNW == 0 || C::WNW % TBLK == 0, "T split");
  const int t_first = ALL_T ? wn * TPW : wn % TBLKX;  // first T block of this wave
  const bool t_wave = RB > 0 && (ALL_T || (wn / TBLKX) == (wm % TG));

  f32x16_t acc[C::NI][C::MJ];
#pragma unroll
  for (int i = 0; i < C::NI; ++i)
#pragma unroll
    for (int j = 0; j < C::MJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  constexpr int TPWX = TPW > 0 ? TPW : 1;
  f32x16_t acct[TPWX];
#pragma unroll
  for (int q = 0; q < TPWX; ++q)
#pragma unroll
    for (int v = 0; v < 16; ++v) acct[q][v] = 0.f;
  int tj[TPWX], trb[TPWX];
#pragma unroll
  for (int q = 0; q < TPWX; ++q) {
    const int b = t_first + q;
    tj[q] = b % C::MJ;
    trb[q] = b / C::MJ;
  }

  // Fragments of one 16-wide k step: x rows (MFMA B operand), W rows and rank-A rows
  // (A operand). `do_t` (a compile-time bool) selects the rank-A part.
  struct Frags {
    u32x4_t x[C::MJ];
    u32x4_t w[C::NI];
    u32x4_t a[TPWX];
    u32x4_t xt[ALL_T ? 1 : TPWX];  // x rows of the T block (read directly when not all waves do T)
  };
  // TN fragment: 32 columns from fbase, k = 16 kk + 8 (lane / 32) + 0..7 of a [64][cols]
  // tile: two transposing reads, rows kb .. kb + 3 and kb + 4 .. kb + 7
  auto tn_frag = [&](const char* tile, int cols, int fbase, int kk) {
    const int g = lane >> 4, i16 = lane & 15;
    const int row = kk * 16 + 8 * (g >> 1) + (i16 >> 2);
    const int f = fbase + 16 * (g & 1) + 4 * (i16 & 3);
    const int off = row * cols * 2 + (((f >> 3) ^ ((row & 3) << 2)) << 4) + (f & 7) * 2;
    const uint2 lo = lds_read_tr8(tile, off), hi = lds_read_tr8(tile, off + 4 * cols * 2);
    return u32x4_t{lo.x, lo.y, hi.x, hi.y};
  };
  auto frag_load = [&](auto do_t, int stage, int kk, Frags& f) {
    const char* sx = lds + stage * STAGE;
    const char* sw = sx + C::XB;
    const char* sa = sw + C::WB;
    if constexpr (TN) {
#pragma unroll
      for (int j = 0; j < C::MJ; ++j) f.x[j] = tn_frag(sx, C::BM, wm * C::TM + j * 32, kk);
#pragma unroll
      for (int i = 0; i < C::NI; ++i) f.w[i] = tn_frag(sw, C::BN, wn * C::TN + i * 32, kk);
      return;
    }
    const int c = kk * 2 + lh;
#pragma unroll
    for (int j = 0; j < C::MJ; ++j) f.x[j] = lds_read16(sx, lds_off(wm * C::TM + j * 32 + l32, c));
    if constexpr (WT) {
#pragma unroll
      for (int i = 0; i < C::NI; ++i) f.w[i] = tn_frag(sw, C::BN, wn * C::TN + i * 32, kk);
    } else if constexpr (HAS_W) {
#pragma unroll
      for (int i = 0; i < C::NI; ++i) f.w[i] = lds_read16(sw, lds_off(wn * C::TN + i * 32 + l32, c));
    }
    if constexpr (decltype(do_t)::value) {
#pragma unroll
      for (int q = 0; q < TPW; ++q) {
        f.a[q] = lds_read16(sa, lds_off(trb[q] * 32 + l32, c));
        if constexpr (!ALL_T) f.xt[q] = lds_read16(sx, lds_off(wm * C::TM + tj[q] * 32 + l32, c));
      }
    }
  };
  auto frag_mma = [&](auto do_t, const Frags& f) {
    if constexpr (HAS_W) {
#pragma unroll
      for (int i = 0; i < C::NI; ++i)
#pragma unroll
        for (int j = 0; j < C::MJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(f.w[i]), as_bf16x8(f.x[j]), acc[i][j], 0, 0, 0);
    }
    if constexpr (decltype(do_t)::value) {
#pragma unroll
      for (int q = 0; q < TPW; ++q) {
        u32x4_t xt;
        if constexpr (ALL_T) {
          xt = f.x[0];
#pragma unroll
          for (int j = 1; j < C::MJ; ++j) xt = (tj[q] == j) ? f.x[j] : xt;  // whole-vector select
        } else {
          xt = f.xt[q];
        }
        acct[q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(f.a[q]), as_bf16x8(xt), acct[q], 0, 0, 0);
      }
    }
  };

  // Interleave the MFMAs of the current k step with the LDS reads of the next one, so
  // the reads are issued early and their latency hides behind the MFMAs (left to
  // itself the scheduler sinks each read next to its use).
  // t_mma: this step's MFMAs include the rank work; t_load: the next step's reads do.
  auto interleave = [&](auto t_mma, auto t_load) {
    constexpr int TTM = decltype(t_mma)::value ? TPW : 0;
    constexpr int TTL = decltype(t_load)::value ? TPW : 0;
    constexpr int NMF = (HAS_W ? C::NI * C::MJ : 0) + TTM;
    constexpr int NRD = (C::MJ + (HAS_W ? C::NI : 0)) * (TN ? 2 : 1) + (WT ? C::NI : 0) + TTL * (ALL_T ? 1 : 2);
    constexpr int PAIRS = NMF < NRD ? NMF : NRD;
#pragma unroll
    for (int q = 0; q < PAIRS; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    if constexpr (NMF > PAIRS) __builtin_amdgcn_sched_group_barrier(0x008, NMF - PAIRS, 0);
    if constexpr (NRD > PAIRS) __builtin_amdgcn_sched_group_barrier(0x100, NRD - PAIRS, 0);
  };

  const int nk = K / BK;
  // The last K tile runs from buffer (nk-1) % NS; the B slice of the LoRA phase is filled
  // into buffer nk % NS, which no later tile uses, while the last tiles run.
  char* lora_t = lds + ((nk - 1) % C::NS) * STAGE;
  char* lora_b = lds + (nk % C::NS) * STAGE;

  constexpr bool RUN_K = HAS_W || RB > 0;
  // Rank work at compile-time k step kc of a K tile: every step with do_t, or only step
  // `cls` (a shared-T class; -1: every step).
  auto t_at = [](auto do_t, auto cls, auto kc) {
    return std::bool_constant<decltype(do_t)::value &&
                              (decltype(cls)::value < 0 || decltype(cls)::value == decltype(kc)::value)>{};
  };
  using K0 = std::integral_constant<int, 0>;
  using KL = std::integral_constant<int, KK - 1>;
  // The K loop, instantiated with and without this wave's T work (`do_t`, at the k steps of
  // `cls`), so the k steps carry no per-step branch and the MFMAs interleave with the next
  // step's LDS reads.
  auto run_k = [&](auto do_t, auto cls) {
    issue(0, 0);
    load_w8(0);
    wait_vm0();
    store_w8(0);
    tn_zero(0, 0);
    ring_barrier();
    WSL_STAMP(srec, 1);
    if (nk > 1) {
      issue(1, BK);
      load_w8(BK);
    }
    if constexpr (LORA) {
      if (nk == 1) issue_b(lora_b, 0);
    }
    Frags cur;
    frag_load(t_at(do_t, cls, K0{}), 0, 0, cur);
    for (int kt = 0; kt < nk; ++kt) {
      const int buf = kt & 1;
      for_ct<0, KK - 1>([&](auto kc) {
        using KN = std::integral_constant<int, decltype(kc)::value + 1>;
        Frags nxt;
        frag_load(t_at(do_t, cls, KN{}), buf, KN::value, nxt);
        frag_mma(t_at(do_t, cls, kc), cur);
        interleave(t_at(do_t, cls, kc), t_at(do_t, cls, KN{}));
        cur = nxt;
      });
      if (kt + 1 < nk) {
        wait_vm0();          // tile kt+1 has landed (the only fill in flight)
        store_w8(buf ^ 1);   // fp8 base: decoded tile kt+1 into its buffer
        tn_zero(buf ^ 1, (kt + 1) * BK);
        ring_barrier();      // all fragments of tile kt are read; tile kt+1 visible
      }
      // One code path for the last k step of every tile keeps the accumulators in one
      // register class (after the last tile its read of the idle buffer is discarded).
      // The fill of tile kt+2 goes out after these MFMAs, so the MFMA pipes restart at
      // once after the barrier.
      Frags nxt;
      frag_load(t_at(do_t, cls, K0{}), buf ^ 1, 0, nxt);
      frag_mma(t_at(do_t, cls, KL{}), cur);
      interleave(t_at(do_t, cls, KL{}), t_at(do_t, cls, K0{}));
      cur = nxt;
      if (kt + 1 < nk) {
        if (kt + 2 < nk) {
          issue(buf, (kt + 2) * BK);
          load_w8((kt + 2) * BK);
        } else if constexpr (LORA) {
          issue_b(lora_b, 0);  // kt + 2 == nk: buffer `buf` is lora_b
        }
      }
    }
    __syncthreads();  // every wave is done with the ring before the LDS is reused
  };
  // The deep ring (NS > 2 buffers: the 128 x 128 tile and the one-wave 128 x 256 tile, at
  // one workgroup per CU): NS K tiles
  // are in flight from the start, and the fill of tile kt+NS goes into tile kt's buffer
  // once every wave has read it (the barrier in tile kt). Each wait leaves the fills of the
  // NS-2 younger tiles in flight. With a workgroup alone on its CU, two buffers left every
  // K tile waiting one fill's latency (about 1.2 us per 128 x 128 x 64 tile at M = 256).
  auto run_k_deep = [&](auto do_t, auto cls) {
    constexpr int NS = C::NS;
    constexpr int PT = C::NXI + (WDIRECT ? C::NWI : 0);  // fills per K tile of every wave (waves < NAI add one)
    const int pre = nk < NS ? nk : NS;
    for (int q = 0; q < pre; ++q) issue(q, q * BK);
    if constexpr (LORA) {
      if (nk < NS) issue_b(lora_b, 0);  // buffer nk is never filled with a K tile
    }
    if (nk >= NS) wait_vm<(NS - 1) * PT>();  // tile 0 has landed
    else wait_vm0();
    ring_barrier();
    WSL_STAMP(srec, 1);
    Frags cur;
    frag_load(t_at(do_t, cls, K0{}), 0, 0, cur);
    int buf = 0;
    for (int kt = 0; kt < nk; ++kt) {
      const int nbuf = buf + 1 == NS ? 0 : buf + 1;
      for_ct<0, KK - 1>([&](auto kc) {
        using KN = std::integral_constant<int, decltype(kc)::value + 1>;
        Frags nxt;
        frag_load(t_at(do_t, cls, KN{}), buf, KN::value, nxt);
        frag_mma(t_at(do_t, cls, kc), cur);
        interleave(t_at(do_t, cls, kc), t_at(do_t, cls, KN{}));
        cur = nxt;
      });
      if (kt + 1 < nk) {
        if (kt + NS - 1 < nk) wait_vm<(NS - 2) * PT>();  // tile kt+1 has landed
        else wait_vm0();
        ring_barrier();  // all fragments of tile kt are read; tile kt+1 visible
      }
      Frags nxt;
      frag_load(t_at(do_t, cls, K0{}), nbuf, 0, nxt);
      frag_mma(t_at(do_t, cls, KL{}), cur);
      interleave(t_at(do_t, cls, KL{}), t_at(do_t, cls, K0{}));
      cur = nxt;
      if (kt + NS < nk) {
        issue(buf, (kt + NS) * BK);
      } else if constexpr (LORA) {
        if (kt + NS == nk) issue_b(lora_b, 0);  // buffer `buf` is lora_b
      }
      buf = nbuf;
    }
    __syncthreads();
  };
  auto run = [&](auto do_t, auto cls) {
    if constexpr (C::NS == 2) run_k(do_t, cls);
    else run_k_deep(do_t, cls);
  };
  using EVERY = std::integral_constant<int, -1>;
  if constexpr (RUN_K) {
    if constexpr (RB == 0) {
      run(std::false_type{}, EVERY{});
    } else if constexpr (PER && !t_here) {
      run(std::false_type{}, EVERY{});
    } else if constexpr (SKT) {
      static_assert(kShareClasses == 4, "shared-T classes are the four k steps of a K tile");
      if (!t_wave || skt_cls < 0) run(std::false_type{}, EVERY{});
      else if (skt_cls == 0) run(std::true_type{}, std::integral_constant<int, 0>{});
      else if (skt_cls == 1) run(std::true_type{}, std::integral_constant<int, 1>{});
      else if (skt_cls == 2) run(std::true_type{}, std::integral_constant<int, 2>{});
      else run(std::true_type{}, std::integral_constant<int, 3>{});
    } else if constexpr (ALL_T) {
      run(std::true_type{}, EVERY{});
    } else {
      if (t_wave) run(std::true_type{}, EVERY{});
      else run(std::false_type{}, EVERY{});
    }
  } else if constexpr (LORA) {
    issue_b(lora_b, 0);
  }
  WSL_STAMP(srec, 2);

  if constexpr (SKT) {
    // Shared T: publish this tile's class, wait for every class of the row block, sum them
    // in class order into acct. Records are lane-major 8-byte words (two accumulators
    // each), one [8][64] block per wave, for every (rbg, class).
    constexpr int CL = kShareClasses;
    static_assert(TPW == 1, "shared T: one T block per T wave");
    auto part_of = [&](int c) { return red_part + (((int64_t)skt_rbg * CL + c) * C::NW + wave) * (8 * 64) + lane; };
    unsigned* const pub = red_cnt + 2 * skt_rbg;  // the arrivals; pub + 1 counts the passes (skt_pass)
    // broadcast word: the W area of the buffer the last K tile ran from (idle now; T is
    // parked below its first BM rows)
    volatile int* skt_seen = reinterpret_cast<volatile int*>(lora_t + C::XB);
    if (skt_cls >= 0) {
      if (t_wave) {
        uint64_t* dst = part_of(skt_cls);
#pragma unroll
        for (int v = 0; v < 8; ++v)
          __hip_atomic_store(dst + v * 64,
                             (uint64_t)__float_as_uint(acct[0][2 * v]) |
                                 ((uint64_t)__float_as_uint(acct[0][2 * v + 1]) << 32),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      wait_vm0();  // the class is out before the arrival
      __syncthreads();
    }
    if (tid == 0) {
      int seen = 0;
      // a publisher that arrives last has seen every class arrive before its own
      if (skt_cls >= 0)
        seen = __hip_atomic_fetch_add(pub, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(CL - 1) &&
               skt_spin > 0;
      for (int it = 0; !seen && it < skt_spin; ++it) {
        if (__hip_atomic_load(pub, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= (unsigned)CL) {
          seen = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      *skt_seen = seen;
    }
    __syncthreads();
    const bool seen = *skt_seen != 0;
    if (t_wave) {
      if (seen) {
        uint64_t w[CL][8];
#pragma unroll
        for (int c = 0; c < CL; ++c)
#pragma unroll
          for (int v = 0; v < 8; ++v)
            w[c][v] = __hip_atomic_load(const_cast<uint64_t*>(part_of(c) + v * 64), __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          float lo = __uint_as_float((uint32_t)w[0][v]), hi = __uint_as_float((uint32_t)(w[0][v] >> 32));
#pragma unroll
          for (int c = 1; c < CL; ++c) {
            lo += __uint_as_float((uint32_t)w[c][v]);
            hi += __uint_as_float((uint32_t)(w[c][v] >> 32));
          }
          acct[0][2 * v] = lo;
          acct[0][2 * v + 1] = hi;
        }
      } else {
        // Every class from global memory: the fragments the K loop reads from LDS (A rows
        // past r read row r - 1, x rows past M row M - 1), the same k steps in the same order.
        const uint16_t* arow = a + (int64_t)min(trb[0] * 32 + l32, r - 1) * lda + lh * 8;
        const uint16_t* xrow = x + (int64_t)min(m0 + wm * C::TM + tj[0] * 32 + l32, M - 1) * ldx + lh * 8;
        f32x16_t tc[CL];
#pragma unroll
        for (int c = 0; c < CL; ++c)
#pragma unroll
          for (int v = 0; v < 16; ++v) tc[c][v] = 0.f;
        for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
          for (int c = 0; c < CL; ++c) {
            const int k = kt * BK + c * 16;
            tc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(ld_global_16(arow + k)),
                                                             as_bf16x8(ld_global_16(xrow + k)), tc[c], 0, 0, 0);
          }
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float t = tc[0][v];
#pragma unroll
          for (int c = 1; c < CL; ++c) t += tc[c][v];
          acct[0][v] = t;
        }
      }
    }
  }

  // ---- per-output-channel dequantisation scale (fp8 base; WT applied it when decoding) ----
  if constexpr (W8 && !WT) {
#pragma unroll
    for (int i = 0; i < C::NI; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int n = n0 + wn * C::TN + i * 32 + g * 8 + lh * 4 + e;
          const float sc = w_scale[map_row(min(n, N - 1), wmap)];
#pragma unroll
          for (int j = 0; j < C::MJ; ++j) acc[i][j][g * 4 + e] *= sc;
        }
      }
    }
  }

  // ---- LoRA up-projection: acc[n][m] += sum_j B[n][j] * T[m][j] in 64-rank chunks ----
  if constexpr (LORA) {
    char* st = PER ? lds + C::NS * STAGE : lora_t;  // T chunk [BM m][64 ranks] (the T region with PER)
    char* sb = lora_b;                   // B chunk [BN n][64 ranks]
    if constexpr (RB > 0) {
      if (t_wave && t_here) {
        // park bf16(s * T): rows wm*TM + tj*32 + l32, ranks trb*32 + 8g + 4*lh + e. Ranks
        // >= r (A rows past r were filled with row r-1) are zeroed here: they meet finite
        // stand-in columns of B in the up-projection.
#pragma unroll
        for (int q = 0; q < TPW; ++q) {
          const int mrow = wm * C::TM + tj[q] * 32 + l32;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int rk = trb[q] * 32 + g * 8 + lh * 4;
            float t4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) t4[e] = rk + e < r ? s * acct[q][g * 4 + e] : 0.f;
            uint2 v;
            v.x = pack_bf16x2(t4[0], t4[1]);
            v.y = pack_bf16x2(t4[2], t4[3]);
            *reinterpret_cast<uint2*>(st + t_off(mrow, trb[q] * 4 + g) + lh * 8) = v;
          }
        }
      }
    }
    const int nrc = (r + 63) / 64;
    for (int rc = 0; rc < nrc; ++rc) {
      const int rk0 = rc * 64;
      if (rc > 0) issue_b(sb, rk0);
      if constexpr (EXT_T) {
        constexpr int TCH = C::BM * 8 / NT;
#pragma unroll
        for (int i = 0; i < TCH; ++i) {
          const int id = i * NT + tid;
          const int row = id >> 3, kr = rk0 + (id & 7) * 8;
          const u32x4_t v = (kr < r) ? ld_global_16(tg + (int64_t)min(m0 + row, M - 1) * ldt + kr) : zero_u32x4();
          lds_write16(st, lds_off(row, id & 7), v);
        }
      }
      wait_vm0();
      __syncthreads();
      const int rem = r - rk0;
      const int nkk = rem >= 64 ? 4 : (rem + 15) / 16;
      for (int kk = 0; kk < nkk; ++kk) {
        const int c = kk * 2 + lh;
        bf16x8_t tf[C::MJ], bf[C::NI];
#pragma unroll
        for (int j = 0; j < C::MJ; ++j) tf[j] = as_bf16x8(lds_read16(st, t_off(wm * C::TM + j * 32 + l32, c)));
#pragma unroll
        for (int i = 0; i < C::NI; ++i) bf[i] = as_bf16x8(lds_read16(sb, lds_off(wn * C::TN + i * 32 + l32, c)));
#pragma unroll
        for (int i = 0; i < C::NI; ++i)
#pragma unroll
          for (int j = 0; j < C::MJ; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[i], tf[j], acc[i][j], 0, 0, 0);
      }
      __syncthreads();
    }
  }

  WSL_STAMP(srec, 3);
  if constexpr (RED) {
    // This split's output partial (its K part of the base product and of the LoRA term, the
    // latter through its own part of T: the up-projection is linear in T) as lane-major
    // 8-byte words, two accumulators each; agent-scope stores, so the reducing workgroup
    // (on any XCD) reads them from memory rather than from a stale L2 line.
    constexpr int EB = C::NI * C::MJ * 8;
    const int S = (int)gridDim.y;
    const int own = (int)blockIdx.y;
    const int64_t first = (int64_t)blockIdx.x * S;  // the tile's split 0 record
    auto rec = [&](int q) { return red_part + ((first + q) * C::NW + wave) * (int64_t)(EB * 64) + lane; };
    {
      uint64_t* dst = rec(own);
#pragma unroll
      for (int i = 0; i < C::NI; ++i)
#pragma unroll
        for (int j = 0; j < C::MJ; ++j)
#pragma unroll
          for (int v = 0; v < 8; ++v)
            __hip_atomic_store(dst + ((i * C::MJ + j) * 8 + v) * 64,
                               (uint64_t)__float_as_uint(acc[i][j][2 * v]) |
                                   ((uint64_t)__float_as_uint(acc[i][j][2 * v + 1]) << 32),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // the flag goes in the ring (idle: the up-projection's last barrier ended its use)
    volatile int* red_last = reinterpret_cast<volatile int*>(lds);
    wait_vm0();  // the record is out before the arrival
    __syncthreads();
    if (tid == 0) {
      const unsigned old = __hip_atomic_fetch_add(red_cnt + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = old == (unsigned)(S - 1);
      if (last) __hip_atomic_store(red_cnt + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *red_last = last ? 1 : 0;
    }
    __syncthreads();
    const bool last = *red_last != 0;
    __syncthreads();  // every wave has the flag before the output staging reuses its word
    if (!last) return;
    // the last split: every split's partial in split order, its own from the registers
    // (the same values it stored), the others' one record's words in flight at a time
    f32x16_t sum[C::NI][C::MJ];
    for (int q = 0; q < S; ++q) {
      f32x16_t part[C::NI][C::MJ];
      if (q == own) {
#pragma unroll
        for (int i = 0; i < C::NI; ++i)
#pragma unroll
          for (int j = 0; j < C::MJ; ++j) part[i][j] = acc[i][j];
      } else {
        const uint64_t* src = rec(q);
        uint64_t wb[EB];
#pragma unroll
        for (int e = 0; e < EB; ++e)
          wb[e] = __hip_atomic_load(const_cast<uint64_t*>(src + e * 64), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int i = 0; i < C::NI; ++i)
#pragma unroll
          for (int j = 0; j < C::MJ; ++j)
#pragma unroll
            for (int v = 0; v < 8; ++v) {
              const uint64_t u = wb[(i * C::MJ + j) * 8 + v];
              part[i][j][2 * v] = __uint_as_float((uint32_t)u);
              part[i][j][2 * v + 1] = __uint_as_float((uint32_t)(u >> 32));
            }
      }
#pragma unroll
      for (int i = 0; i < C::NI; ++i)
#pragma unroll
        for (int j = 0; j < C::MJ; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) sum[i][j][v] = q == 0 ? part[i][j][v] : sum[i][j][v] + part[i][j][v];
    }
#pragma unroll
    for (int i = 0; i < C::NI; ++i)
#pragma unroll
      for (int j = 0; j < C::MJ; ++j) acc[i][j] = sum[i][j];
  }

  if constexpr (SPLIT) {
    // fp32 partials straight from the accumulators: lane pairs (lh) cover 8 consecutive
    // n of one row, the four groups g a whole 128-byte line, merged in L2.
    float* yf = reinterpret_cast<float*>(y) + (int64_t)blockIdx.y * M * ldy;
#pragma unroll
    for (int j = 0; j < C::MJ; ++j) {
      const int m = m0 + wm * C::TM + j * 32 + l32;
      if (m >= M) continue;
#pragma unroll
      for (int i = 0; i < C::NI; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + wn * C::TN + i * 32 + g * 8 + lh * 4;  // N % 8 == 0: n < N covers n + 3
          if (n < N)
            *reinterpret_cast<f32x4_t*>(yf + (int64_t)m * ldy + n) =
                f32x4_t{acc[i][j][g * 4 + 0], acc[i][j][g * 4 + 1], acc[i][j][g * 4 + 2], acc[i][j][g * 4 + 3]};
        }
      }
    }
    return;
  }

  // SKT: this tile is past its reads of the classes (they returned before T was parked);
  // the row block's last tile to pass returns both counters to zero. Thread 0 waits for the
  // counter's round trip after its stores are issued, where nothing waits on it.
  auto skt_pass = [&]() {
    if constexpr (SKT) {
      if (tid == 0) {
        unsigned* const pub = red_cnt + 2 * skt_rbg;
        const unsigned old = __hip_atomic_fetch_add(pub + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == (unsigned)(skt_ntiles - 1)) {
          __hip_atomic_store(pub, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(pub + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  };

  // ---- store. The accumulators hold 4 consecutive n of one m per lane and group, i.e.
  // 16-byte pieces of 32 different rows per wave instruction; written straight to y
  // they reach L2 as partial lines. The tile is staged through LDS (row stride OS) and
  // written back row-contiguously, 16 bytes per lane.
  char* ot = lds;  // the ring is idle: the last barrier above ended every LDS use
#pragma unroll
  for (int j = 0; j < C::MJ; ++j) {
    const int mr = wm * C::TM + j * 32 + l32;
    float keep = yscale;
    if constexpr (GATHER) {
      const int64_t id = gidx[min(m0 + mr, M - 1)];
      if (id < 0 || id >= grows) keep = 0.f;  // out-of-range ids give zero rows
    }
#pragma unroll
    for (int i = 0; i < C::NI; ++i) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int nc = wn * C::TN + i * 32 + g * 8 + lh * 4;
        const f32x16_t& cc = acc[i][j];
        uint2 v;
        v.x = pack_bf16x2(keep * cc[g * 4 + 0], keep * cc[g * 4 + 1]);
        v.y = pack_bf16x2(keep * cc[g * 4 + 2], keep * cc[g * 4 + 3]);
        *reinterpret_cast<uint2*>(ot + mr * OS + nc * 2) = v;
      }
    }
  }
  __syncthreads();
  WSL_STAMP(srec, 4);
  constexpr int CPR = C::BN / 8;  // 16-byte chunks per tile row
  const bool a16 = ((reinterpret_cast<uintptr_t>(y) & 15u) == 0) && ((ldy & 7) == 0);
  if (a16 && m0 + C::BM <= M && n0 + C::BN <= N) {
    // whole tile in range: every LDS read first, then the stores, with no per-chunk tests.
    // The stores are non-temporal: y is written once and not read by this launch, and
    // streamed past the caches it leaves the lines the next launch reads in place (same
    // box, config 2: 871 -> 902 TFLOP/s one launch per projection, 877 -> 960 grouped,
    // where a temporal 64-96 MB output slowed the following launch by ~25 %).
    constexpr int IT = C::BM * CPR / NT;
    static_assert(C::BM * CPR % NT == 0, "store split");
    u32x4_t v[IT];
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int q = i * NT + tid;
      v[i] = *reinterpret_cast<const u32x4_t*>(ot + (q / CPR) * OS + (q % CPR) * 16);
    }
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int q = i * NT + tid;
      store_y16(v[i], reinterpret_cast<u32x4_t*>(y + (int64_t)(m0 + q / CPR) * ldy + n0 + (q % CPR) * 8));
    }
    WSL_STAMP(srec, 5);
    skt_pass();
    return;
  }
#pragma unroll 4
  for (int q = tid; q < C::BM * CPR; q += NT) {
    const int row = q / CPR, c = q % CPR;
    const int m = m0 + row, n = n0 + c * 8;
    if (m >= M || n >= N) continue;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ot + row * OS + c * 16);
    uint16_t* dst = y + (int64_t)m * ldy + n;
    if (n + 8 <= N) {
      if (a16) {
        store_y16(v, reinterpret_cast<u32x4_t*>(dst));
      } else {
        reinterpret_cast<uint2*>(dst)[0] = uint2{v[0], v[1]};
        reinterpret_cast<uint2*>(dst)[1] = uint2{v[2], v[3]};
      }
    } else {
      for (int e = 0; e < N - n; ++e) dst[e] = (uint16_t)(v[e >> 1] >> ((e & 1) * 16));
    }
  }
  WSL_STAMP(srec, 5);
  skt_pass();
  };  // do_tile

  if constexpr (PER) {
    // The first tile (with T) peeled from the rest: the loop then holds only the K loop
    // without rank work. After each tile every wave has read its share of the staged output
    // before the next tile's fills land in the ring (the stores stay in flight).
    do_tile(0, std::true_type{});
    ring_barrier();
    for (int tq = 1; tq < tpw; ++tq) {
      do_tile(tq, std::false_type{});
      ring_barrier();
    }
  } else {
    do_tile(0, std::true_type{});
  }
}

using CfgBig = Cfg<256, 256, 2, 8>;   // 8 waves, 128(n) x 64(m) per wave
using CfgTall = Cfg<128, 256, 4, 8>;  // 8 waves, 64 x 64 per wave
using CfgTall3 = Cfg<128, 256, 4, 8, 3>;  // the same tile on a three-buffer ring (one wave of tiles)
using CfgMid = Cfg<256, 192, 2, 8>;   // 8 waves, 96(n) x 64(m) per wave
using CfgSmall = Cfg<128, 128, 2, 8>;  // 8 waves, 64(n) x 32(m) per wave; also the rank pre-pass (N = r)
using CfgDeep = Cfg<128, 128, 2, 8, 4>;  // the same tile with four ring buffers: one workgroup per CU

// End column of group g of a grouped launch (INT_MAX past the last group: no tile
// starts there).
int group_end(const LoraArgs& p, int g) { return g + 1 < p.groups ? (int)p.gend[g] : INT_MAX; }

// Whether tiles BN wide keep every group of a grouped launch within whole tiles.
bool groups_fit(const LoraArgs& p, int bn) {
  for (int g = 0; g + 1 < p.groups; ++g)
    if (p.gend[g] % bn != 0) return false;
  return true;
}

template <class C, int WDT, bool HAS_W, int RB, bool EXT_T, bool GATHER, bool SPLIT = false, bool TN = false,
          bool RED = false, bool PER = false, bool WT = false, bool SKT = false>
hipError_t launch_cfg(const LoraArgs& p, const uint16_t* tg, int64_t ldt, int splits = 1,
                      uint64_t* red_part = nullptr, unsigned* red_cnt = nullptr, int tpw = 1, int skt_spin = 0) {
  const int tiles_m = (int)((p.M + C::BM - 1) / C::BM);
  const int tiles_n = (int)((p.N + C::BN - 1) / C::BN);
  prefill_kernel<C, WDT, HAS_W, RB, EXT_T, GATHER, SPLIT, TN, RED, PER, WT, SKT>
      <<<dim3(tiles_m * tiles_n / (PER ? tpw : 1), splits), dim3(C::NT), 0, p.stream>>>(
      reinterpret_cast<const uint16_t*>(p.x), p.ldx, p.gather, p.gather_rows, p.w, p.ldw, p.w_scale,
      reinterpret_cast<const uint16_t*>(p.a), p.lda, tg, ldt,
      reinterpret_cast<const uint16_t*>(p.b), p.ldb, p.scale, p.yscale,
      reinterpret_cast<uint16_t*>(p.y), p.ldy, (int)p.M, (int)p.N, (int)p.K, (int)p.r, tiles_m, tiles_n,
      group_end(p, 0), group_end(p, 1), group_end(p, 2), p.groups > 1 ? p.r * p.lda : 0,
      (p.groups > 1 && tg != nullptr) ? (int)p.r : 0, p.wmap, red_part, red_cnt, PER ? tpw : 1, skt_spin);
  return hipGetLastError();
}

// ---- Shared T (the SKT form) ----
// Records of one row block and group: kShareClasses classes x 8 waves x 64 lanes x 8 words.
constexpr size_t kSktRbgBytes = (size_t)kShareClasses * 8 * 64 * 8 * 8;
// Polls of the row block's counter (each a memory round trip and a short sleep, 1 us or
// more) before a tile computes T itself: milliseconds, against the few microseconds the
// tiles of one wave finish apart.
constexpr int kSktSpin = 1 << 12;
// K tiles from which sharing pays: the exchange (the classes out and arrived, the counter
// seen, the classes read: about 3 us with the tiles' skew) against three quarters of T's
// MFMAs (1/9 of the loop's). Alternating graphs of 28 launches, shared against T in every
// tile, two orders on one box: 8192 x 6144 -> 2048 (96 K tiles) 164.0 / 163.2 against
// 172.5 / 173.3 us; 8192 x 3072 -> 1024 (48) 55.4 / 56.2 against 56.8 / 56.2; 8192 x 2048
// -> 2048 (32) 63.1 / 63.4 against 63.5 / 63.6; 8192 x 2048 -> 1024 (32) 40.0 / 40.1
// against 39.5 / 39.3.
constexpr int kSktMinKTiles = 64;

// Row-block groups of a launch of BM x BN tiles that shares T between the column tiles of
// each row block, or 0 where it does not: a long K (kSktMinKTiles), one wave of tiles on
// this device (every workgroup resident at once, so the wait for the other tiles' classes
// is short), at least kShareClasses tiles in every group, the arrival counters, and room in
// the workspace for the records. WSL_OPT_PREFILL_SHARED_T = -1 keeps T in every tile; 2
// drops the K bound (side-by-side timing of the shorter launches).
int64_t shared_t_rbgs(const LoraArgs& p, int bm, int bn) {
  const int64_t opt = option(WSL_OPT_PREFILL_SHARED_T);
  if (opt < 0 || p.red_cnt == nullptr || p.ws == nullptr) return 0;
  if (p.K / BK < kSktMinKTiles && opt != 2) return 0;
  const int64_t tiles_m = (p.M + bm - 1) / bm, tiles_n = (p.N + bn - 1) / bn;
  const int cus = device_cus();
  if (cus <= 0 || tiles_m * tiles_n > cus) return 0;
  int64_t start = 0;
  for (int g = 0; g < p.groups; ++g) {
    const int64_t end = g + 1 < p.groups ? p.gend[g] : p.N;
    if ((end - start + bn - 1) / bn < kShareClasses) return 0;
    start = end;
  }
  const int64_t rbgs = tiles_m * p.groups;
  if (2 * rbgs > kRedMaxTiles || (size_t)rbgs * kSktRbgBytes > p.ws_bytes) return 0;
  return rbgs;
}

// Workspace bytes the shared-T records of an M x N launch can take: at most a quarter of
// its 128 x 256 tiles are row-block groups (every group has at least four tiles), and only
// when those tiles are one wave on this device.
size_t shared_t_bytes(int64_t M, int64_t N, int64_t K) {
  if (K / BK < kSktMinKTiles && option(WSL_OPT_PREFILL_SHARED_T) != 2) return 0;
  const int64_t tiles = ((M + 127) / 128) * ((N + 255) / 256);
  const int cus = device_cus();
  return (cus > 0 && tiles <= cus) ? (size_t)((tiles + kShareClasses - 1) / kShareClasses) * kSktRbgBytes : 0;
}

template <class C>
hipError_t launch_skt(const LoraArgs& p) {
  const int spin = option(WSL_OPT_PREFILL_SHARED_T) == 1 ? 0 : kSktSpin;
  return launch_cfg<C, kBF16, true, 1, false, false, false, false, false, false, false, true>(
      p, nullptr, 0, 1, reinterpret_cast<uint64_t*>(p.ws), p.red_cnt, 1, spin);
}

// Column tiles per persistent strip for a launch of BM x BN tiles, or 1 (one tile per
// workgroup). Strips are taken where the tiles are a whole number k >= 2 of waves over the
// 256 CUs: 256 workgroups then run k tiles each, and T, computed in the first, costs one
// tile's rank MFMAs instead of k. A strip stays in one row of tiles and one group.
// WSL_OPT_PREFILL_STRIPS = -1 keeps one tile per workgroup (side-by-side timing).
int strip_tiles(const LoraArgs& p, int bm, int bn) {
  if (option(WSL_OPT_PREFILL_STRIPS) < 0) return 1;
  const int64_t tiles_m = (p.M + bm - 1) / bm, tiles_n = (p.N + bn - 1) / bn;
  const int64_t tiles = tiles_m * tiles_n;
  if (tiles < 512 || tiles % 256 != 0) return 1;
  const int64_t k = tiles / 256;
  if (k > tiles_n || tiles_n % k != 0) return 1;
  for (int g = 0; g + 1 < p.groups; ++g)
    if (p.gend[g] % (k * bn) != 0) return 1;
  return (int)k;
}

// One tile configuration's launch: persistent strips of `strips` tiles (bf16 W with T
// computed in the kernel, two-buffer ring), or one tile per workgroup. 128 x 256 tiles
// without strips (config 2's o and down: one tile per CU) run on a three-buffer ring, two K
// tiles in flight, where a rank block leaves room for it (156 KB of LDS): same box,
// alternating, o 41.1 / 41.3 against 41.8 / 42.0 us and down 56.5 / 56.4 against 58.9 /
// 57.6.
template <class C, int WDT, bool HAS_W, int RB, bool EXT_T, bool GATHER, bool WT = false>
hipError_t launch_tiles(const LoraArgs& p, const uint16_t* tg, int64_t ldt, int strips) {
  constexpr bool SKT_FORM = WDT == kBF16 && HAS_W && RB == 1 && !EXT_T && !GATHER && !WT;
  if constexpr (std::is_same_v<C, CfgTall> && WDT == kBF16 && !GATHER && RB <= 1) {
    if (strips <= 1) {
      if constexpr (SKT_FORM) {
        if (shared_t_rbgs(p, CfgTall3::BM, CfgTall3::BN) > 0) return launch_skt<CfgTall3>(p);
      }
      return launch_cfg<CfgTall3, WDT, HAS_W, RB, EXT_T, GATHER, false, false, false, false, WT>(p, tg, ldt);
    }
  }
  if constexpr (std::is_same_v<C, CfgBig> && SKT_FORM) {
    if (strips <= 1 && shared_t_rbgs(p, C::BM, C::BN) > 0) return launch_skt<CfgBig>(p);
  }
  if constexpr (WDT == kBF16 && HAS_W && RB > 0 && !EXT_T && !GATHER && C::NS == 2) {
    if (strips > 1)
      return launch_cfg<C, WDT, HAS_W, RB, EXT_T, GATHER, false, false, false, true, WT>(p, tg, ldt, 1, nullptr,
                                                                                         nullptr, strips);
  }
  return launch_cfg<C, WDT, HAS_W, RB, EXT_T, GATHER, false, false, false, false, WT>(p, tg, ldt);
}

// Fraction of the 256 CUs kept busy over the launch's waves of workgroups.
double wave_efficiency(int64_t tiles) {
  const int64_t waves = (tiles + 255) / 256;
  return (double)tiles / (double)(waves * 256);
}

// Tile configuration by how well its tiles fill the CUs, discounted by its measured
// in-loop efficiency relative to 256 x 256 (smaller wave tiles read more LDS per MFMA).
// 128 x 128 on a full chip: 0.81 of 256 x 256 at M = N = 8192, K = 4096, 0.75 at
// M = N = K = 4096; it wins where the larger tiles leave CUs idle (M = 4096, N = 1024:
// 256 tiles against 128 of 128 x 256, 642 against 552 TFLOP/s).
// kDeep is the 128 x 128 tile on the four-buffer ring.
enum class Tile { kBig, kMid, kTall, kSmall, kDeep };
// A grouped launch only considers configurations whose tile width divides every group
// boundary (one of 256 and 128 always does: prefill_groups_supported checks it).
// no_mid: the token-major W' tile of the input gradient needs whole 128-column chunks.
Tile choose_tile(const LoraArgs& p, bool no_mid = false) {
  const int64_t tm = (p.M + 255) / 256;
  const bool f256 = groups_fit(p, 256), f192 = groups_fit(p, 192) && !no_mid, f128 = groups_fit(p, 128);
  const double big = f256 ? wave_efficiency(tm * ((p.N + 255) / 256)) : -1.0;
  const double mid = f192 ? wave_efficiency(tm * ((p.N + 191) / 192)) * 0.95 : -1.0;
  const double tall = f256 ? wave_efficiency(((p.M + 127) / 128) * ((p.N + 255) / 256)) * 0.85 : -1.0;
  const double small = f128 ? wave_efficiency(((p.M + 127) / 128) * ((p.N + 127) / 128)) * 0.75 : -1.0;
  if (small > big && small > mid && small > tall) return Tile::kSmall;
  if (mid > big && mid > tall) return Tile::kMid;
  return tall > big ? Tile::kTall : Tile::kBig;
}

int tile_rows(Tile t) { return (t == Tile::kBig || t == Tile::kMid) ? 256 : 128; }
int tile_cols(Tile t) { return t == Tile::kMid ? 192 : (t == Tile::kSmall || t == Tile::kDeep) ? 128 : 256; }

// The tile loop's configuration for a launch of the K loop with RB in-loop rank blocks
// (ext_t: T from the pre-pass), and its persistent strip length.
struct TilePick {
  Tile tile;
  int strips;
};
TilePick pick_tiles(const LoraArgs& p, int wdt, bool has_w, int rb, bool ext_t, bool gather, bool wt = false) {
  TilePick t{Tile::kBig, 1};
  if (rb == 2) {
    // Ranks 33-64 (two rank blocks) use 128 x 256, whose 64 x 64 wave tile leaves registers
    // for the second block's T accumulators beside the base accumulators, or 128 x 128 (one
    // rank block per wave) where the wider tiles would leave more CUs idle.
    const int64_t tm = (p.M + 127) / 128;
    const double tall = wave_efficiency(tm * ((p.N + 255) / 256)) * 0.85;  // groups fit 256 (checked)
    const double small = wave_efficiency(tm * ((p.N + 127) / 128)) * 0.75;
    t.tile = small > tall ? Tile::kSmall : Tile::kTall;
  } else {
    t.tile = choose_tile(p, wt);
  }
  // 128 x 128 tiles: with at most one workgroup per CU (no more tiles than CUs) the deep
  // ring, else two workgroups per CU on the two-buffer ring (they hide each other's fills).
  if (t.tile == Tile::kSmall && wdt == kBF16 && !gather && ((p.M + 127) / 128) * ((p.N + 127) / 128) <= 256)
    t.tile = Tile::kDeep;
  if (wdt == kBF16 && has_w && rb > 0 && !ext_t && !gather && t.tile != Tile::kSmall && t.tile != Tile::kDeep)
    t.strips = strip_tiles(p, tile_rows(t.tile), tile_cols(t.tile));
  return t;
}

template <int WDT, bool HAS_W, int RB, bool EXT_T, bool GATHER = false, bool WT = false>
hipError_t launch_variant(const LoraArgs& p, const uint16_t* tg, int64_t ldt) {
  const TilePick t = pick_tiles(p, WDT, HAS_W, RB, EXT_T, GATHER, WT);
  if constexpr (WDT == kBF16 && !GATHER) {
    if (t.tile == Tile::kDeep)
      return launch_cfg<CfgDeep, WDT, HAS_W, RB, EXT_T, GATHER, false, false, false, false, WT>(p, tg, ldt);
  }
  if constexpr (RB == 2) {
    if (t.tile == Tile::kTall) return launch_tiles<CfgTall, WDT, HAS_W, RB, EXT_T, GATHER, WT>(p, tg, ldt, t.strips);
    return launch_cfg<CfgSmall, WDT, HAS_W, RB, EXT_T, GATHER, false, false, false, false, WT>(p, tg, ldt);
  } else {
    switch (t.tile) {
      case Tile::kMid:
        if constexpr (!WT) return launch_tiles<CfgMid, WDT, HAS_W, RB, EXT_T, GATHER>(p, tg, ldt, t.strips);
        else return hipErrorInvalidValue;  // not picked for WT (no_mid)
      case Tile::kTall: return launch_tiles<CfgTall, WDT, HAS_W, RB, EXT_T, GATHER, WT>(p, tg, ldt, t.strips);
      case Tile::kSmall:
      case Tile::kDeep:
        return launch_cfg<CfgSmall, WDT, HAS_W, RB, EXT_T, GATHER, false, false, false, false, WT>(p, tg, ldt);
      default: return launch_tiles<CfgBig, WDT, HAS_W, RB, EXT_T, GATHER, WT>(p, tg, ldt, t.strips);
    }
  }
}

// Whether a launch's T comes from the rank pre-pass instead of its K loop: always above
// RIN; for ranks 33-64 (two in-loop rank blocks, which fit only the 128 x 256 and 128 x 128
// tiles and add a quarter or a half to their MFMAs) wherever T from the pre-pass lets the
// launch take a wider tile than 128 x 128 (1.7B gate|up, r = 64, us per launch in graphs of
// 28, cold weights: M = 8192 406.7 against 515.4 in the loop, 2048 123.2 against 132.5,
// 1024 68.3 against 85.3 (256 x 192 tiles), 512 45.9 against 48.7 (128 x 256 both ways);
// where both ways take 128 x 128 tiles the loop wins: M = 256 28.8 against 35.8, q|k|v at
// 1024 30.3 against 36.7).
bool prepass_rank(const LoraArgs& p) {
  if (p.r > RIN) return true;
  if (p.r <= 32 || p.w == nullptr || p.gather != nullptr) return false;
  const Tile t = pick_tiles(p, (int)p.w_dtype, true, 0, true, false).tile;
  return t != Tile::kSmall && t != Tile::kDeep;
}

// In-loop rank blocks of a launch (0 with T from the pre-pass).
int rank_blocks_of(const LoraArgs& p) {
  if (p.r == 0 || prepass_rank(p)) return 0;
  return p.r <= 32 ? 1 : 2;
}

// tg: T from the pre-pass (prepass_rank), else nullptr and T in the K loop
template <int WDT, bool HAS_W>
hipError_t launch_rank(const LoraArgs& p, const uint16_t* tg, int64_t ldt) {
  if (tg != nullptr) return launch_variant<WDT, HAS_W, 0, true>(p, tg, ldt);
  if (p.r == 0) return launch_variant<WDT, HAS_W, 0, false>(p, nullptr, 0);
  if (p.r <= 32) return launch_variant<WDT, HAS_W, 1, false>(p, nullptr, 0);
  return launch_variant<WDT, HAS_W, 2, false>(p, nullptr, 0);
}

bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

// K splits of the rank pre-pass: enough 128 x 128 tiles to cover the 256 CUs, at least
// kMinSplitTiles K tiles per split, and a divisor of the K tile count so every split has
// the same length (the fp32 sums then do not depend on M).
constexpr int kMaxSplits = 16;
constexpr int kMinSplitTiles = 4;
int rank_splits(int64_t M, int64_t K, int64_t r) {
  const int64_t tiles = ((M + CfgSmall::BM - 1) / CfgSmall::BM) * ((r + CfgSmall::BN - 1) / CfgSmall::BN);
  const int64_t nk = K / BK;
  int64_t want = (256 + tiles - 1) / tiles;
  if (want > kMaxSplits) want = kMaxSplits;
  if (want > nk / kMinSplitTiles) want = nk / kMinSplitTiles;
  for (int64_t s = want; s > 1; --s)
    if (nk % s == 0) return (int)s;
  return 1;
}

// T[m][k] = bf16(s * sum_q part[q][m][k]), q in order: 8 consecutive ranks per thread.
__global__ void __launch_bounds__(256)
rank_reduce_kernel(const float* __restrict__ part, int splits, int64_t slice, float s,
                   uint16_t* __restrict__ t) {
  const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e >= slice) return;
  f32x4_t lo = *reinterpret_cast<const f32x4_t*>(part + e);
  f32x4_t hi = *reinterpret_cast<const f32x4_t*>(part + e + 4);
  for (int q = 1; q < splits; ++q) {
    lo += *reinterpret_cast<const f32x4_t*>(part + q * slice + e);
    hi += *reinterpret_cast<const f32x4_t*>(part + q * slice + e + 4);
  }
  *reinterpret_cast<u32x4_t*>(t + e) = u32x4_t{pack_bf16x2(s * lo[0], s * lo[1]), pack_bf16x2(s * lo[2], s * lo[3]),
                                               pack_bf16x2(s * hi[0], s * hi[1]), pack_bf16x2(s * hi[2], s * hi[3])};
}

}  // namespace

bool groups_fit_tiles(const LoraArgs& p, int bn) { return groups_fit(p, bn); }

// A grouped launch needs the prefill path and group ends that whole tiles of one of the
// configurations its rank takes respect (ranks 33-64 run only on 256-wide tiles).
bool prefill_groups_supported(const LoraArgs& p) {
  if (p.groups < 1 || p.groups > kMaxGroups) return false;
  if (p.groups == 1) return true;
  if (p.r > 32 && p.r <= RIN) return groups_fit(p, 256);
  return groups_fit(p, 256) || groups_fit(p, 192) || groups_fit(p, 128);
}

bool prefill_supported(const LoraArgs& p) {
  if (p.K % BK != 0) return false;
  if (p.M > (int64_t)1 << 30 || p.N > (int64_t)1 << 30 || p.K > (int64_t)1 << 30) return false;
  // 32-bit lane offsets of the direct fills cover a 256-row tile of x and W
  if (p.ldx > ((int64_t)1 << 22) || p.ldw > ((int64_t)1 << 22) || p.lda > ((int64_t)1 << 22)) return false;
  if (!aligned16(p.x) || p.ldx % 8 != 0) return false;
  if (p.wmap.P != 0 && p.wrows * p.ldw * 2 >= ((int64_t)1 << 32)) return false;
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

// Bytes of the rank pre-pass region for M rows of rank rt: T [M][rt] bf16, then, when K is
// split, the fp32 partials [splits][M][rt] at the next 256-byte boundary.
size_t rank_prepass_bytes(int64_t M, int64_t K, int64_t rt) {
  const size_t t_bytes = ((size_t)(M * rt * 2) + 255) & ~(size_t)255;
  const int splits = rank_splits(M, K, rt);
  return t_bytes + (splits > 1 ? (size_t)splits * M * rt * 4 : 0);
}

namespace {
// Which path an fp8 W takes on prefill shapes. Two activation terms on the fp8 matrix cores
// do the MFMA work of the bf16 product and add the activation split (a read and a write of
// x); the fp8 kernel has only 256 x 256 tiles, where the bf16 path also has narrower tiles
// and split forms. They pay where the launch has more 256 x 256 tiles than the 256 CUs;
// narrower launches decode W onto the bf16 matrix cores. Config 5 at M = 4096 (graphs of
// 10 launches, one box; fp8 matrix cores with the split against decoded W): gate (768
// tiles) 353.9 against 371.5 us, q|k|v grouped (384) 235.7 against 249.2, gate|up grouped
// 683.7 against 730.4; q and o (256 tiles) 141.9 / 141.3 against 140.8 / 140.0, down
// (4096 x 12288, the split of a 12288-wide x costing 31 us) 366.2 against 360.8, k and v
// (1024 x 4096, 64 tiles) 116.4 against 68.6. One activation term
// (WSL_DTYPE_FP8_E4M3_ACT8) always takes the fp8 matrix cores. WSL_OPT_FP8_PREFILL = 1
// decodes W for every shape, 2 takes the fp8 matrix cores for every shape.
bool fp8_matrix_cores(const LoraArgs& p) {
  const int64_t o = option(WSL_OPT_FP8_PREFILL);
  if (o == 1 || p.fp8_terms <= 0 || !prefill_fp8_supported(p)) return false;
  if (o == 2 || p.fp8_terms == 1) return true;
  return ((p.M + 255) / 256) * ((p.N + 255) / 256) > 256;
}
}  // namespace

// ---- Medium M: split-K over few row tiles ----
// Just past the decode path (M <= 64) the tile grid has one or two rows of tiles, and each
// workgroup's K loop is a chain of dependent fills with little MFMA work to hide them (at
// M = 65, 2048 x 6144 ran 94 us, W streamed at 0.27 TB/s). Such shapes split K: the base
// product runs as the split-K plain GEMM over 128 x 128 tiles (fp32 partials
// [splits][M][N]), T comes from the rank pre-pass, and a combine kernel sums the partials in
// split order, adds T . B^T and rounds once. The split count depends on M and K, halved
// while the partials exceed their budget; a grouped call whose groups would take another
// count alone goes group by group, so grouped outputs stay those of the single calls.
constexpr int kMediumMaxM = 160;  // measured: the split form wins at M = 65-128, loses at 192-256
// (since the in-launch split-K form, taken first for ranks up to 64, it serves ranks 65-256)
constexpr int kMediumMaxSplits = 16;
constexpr size_t kMediumPartBytes = (size_t)24 << 20;  // with T, within the no-allocation scratch

int medium_splits(int64_t M, int64_t N, int64_t K, int64_t rt, int w_dtype, bool has_w, bool gather) {
  if (!has_w || gather || w_dtype != kBF16 || M > kMediumMaxM || M < 1) return 0;
  if (rt > 256) return 0;  // the combine kernel stages 32 rows of T (all rt ranks) in LDS
  if (option(WSL_OPT_PREFILL_MEDIUM) < 0) return 0;  // the unsplit tiles, for side-by-side timing
  const int64_t nk = K / BK;
  // Since the 128 x 128 tiles' deep ring, the unsplit tiles win below 64 K tiles (rank 128:
  // 100 x 2048 x 2048 27.6 against 30.9 us, 160 x 6144 x 2048 30.6 against 41.6; rank 96,
  // 150 x 3072 x 1024 19.3 against 31.9) and lose above (130 x 2048 x 6144: 60.9 against 41.6)
  if (nk < 64) return 0;
  const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128);
  if (tiles >= 192) return 0;  // enough workgroups without a split
  int s = 1;
  while (s * 2 <= kMediumMaxSplits && nk % (s * 2) == 0 && nk / (s * 2) >= 2) s *= 2;
  while (s > 1 && (size_t)s * M * N * 4 > kMediumPartBytes) s /= 2;
  return s > 1 ? s : 0;
}

// ---- Split-K in one launch (the RED form of prefill_kernel over 128 x 128 tiles) ----
// For shapes whose 128 x 128 tiles leave most CUs idle (few rows of tokens, or narrow N),
// K is cut into S equal parts over a second grid dimension. Each split runs the fused K
// loop (T included) over its part, applies its part of T through B (the up-projection is
// linear in T) and leaves an fp32 record of its output partial; the last split of a tile
// sums the partials in split order (its own from registers) and stores the tile. One
// launch, no pre-pass: T comes from the same K loops. The split count fills at most one workgroup per CU (the deep ring's LDS
// takes a whole CU; allowing two per CU measured the same), keeps at least kRedMinTiles K
// tiles per split, divides the K tile count and keeps the records within their budget (the
// no-allocation scratch holds them).
constexpr int kRedMaxSplits = 16;
constexpr int kRedMinTiles = 8;  // 1.7B layer at M = 129-256: 8 K tiles per split 7-8 % ahead of 4
constexpr size_t kRedPartBytes = (size_t)24 << 20;

// Bytes of one (tile, split) record: 8 waves x 64 lanes x 16 words (the output partial).
size_t red_record_bytes() { return (size_t)CfgDeep::NW * 64 * 8 * (CfgDeep::NI * CfgDeep::MJ * 8); }

int red_splits(int64_t M, int64_t N, int64_t K, int w_dtype, bool has_w, bool gather) {
  if (!has_w || gather || w_dtype != kBF16 || M < 1) return 0;
  const int64_t nk = K / BK;
  const int64_t tiles = ((M + 127) / 128) * ((N + 127) / 128);
  if (tiles > kRedMaxTiles) return 0;
  const int64_t f = option(WSL_OPT_PREFILL_SPLIT);  // off, or a forced split count (side-by-side timing)
  if (f < 0) return 0;
  if (f >= 2 && f <= kRedMaxSplits && nk % f == 0 && (size_t)(tiles * f) * red_record_bytes() <= kRedPartBytes)
    return (int)f;
  // At 97-128 tiles the unsplit launch already covers half the CUs: splitting in two pays
  // from 24 K tiles (1.7B shapes, r = 64, us per launch in graphs of 28, cold weights:
  // M x N x K = 1024 x 2048 x 2048 21.8 against 23.8 unsplit, 896 x 2048 x 2048 21.2 against
  // 23.8, 1024 x 2048 x 1536 18.8 against 19.5; 1024 x 2048 x 1024 16.2 against 14.9 and
  // 2048 x 1024 x 1024 16.0 against 14.9). At 96 tiles (gate|up at 128 tokens) it pays.
  if (tiles > 96 && nk < 24) return 0;
  int s = 1;
  while (s * 2 <= kRedMaxSplits && nk % (s * 2) == 0 && nk / (s * 2) >= kRedMinTiles && tiles * s * 2 <= 256) s *= 2;
  while (s > 1 && (size_t)(tiles * s) * red_record_bytes() > kRedPartBytes) s /= 2;
  return s > 1 ? s : 0;
}

namespace {
hipError_t launch_red(const LoraArgs& p, int splits) {
  LoraArgs q = p;
  q.K = p.K / splits;
  uint64_t* part = reinterpret_cast<uint64_t*>(p.ws);
  if (p.r == 0) return launch_cfg<CfgDeep, kBF16, true, 0, false, false, false, false, true>(q, nullptr, 0, splits, part, p.red_cnt);
  if (p.r <= 32) return launch_cfg<CfgDeep, kBF16, true, 1, false, false, false, false, true>(q, nullptr, 0, splits, part, p.red_cnt);
  return launch_cfg<CfgDeep, kBF16, true, 2, false, false, false, false, true>(q, nullptr, 0, splits, part, p.red_cnt);
}

// y[m][n] = bf16(sum_s part[s][m][n] + sum_j T[m][goff(n) + j] B[n][j]): the partials in split
// order, then the LoRA up-projection over the bf16 T of the rank pre-pass (s applied there).
// A workgroup owns 32 rows x 32 columns: it stages their T rows (all rt ranks) and B rows in
// LDS, and each thread takes 4 consecutive columns of one row (coalesced partials, 8-byte
// stores); lanes of one row read the same T words and lanes of one column quad the same B
// words, so the LDS reads broadcast.
constexpr int MC_ROWS = 32, MC_COLS = 32;
__global__ void __launch_bounds__(256)
medium_combine_kernel(const float* __restrict__ part, int splits, int M, int N, const uint16_t* __restrict__ t,
                      int ldt, const uint16_t* __restrict__ b, int64_t ldb, int r, int ge0, int ge1, int ge2,
                      uint16_t* __restrict__ y, int64_t ldy) {
  // LDS rows padded by one word: the 8 rows (T) or column quads (B) a wave reads at once
  // then fall on different banks instead of one
  extern __shared__ __attribute__((aligned(16))) uint32_t mc_lds[];
  const int tsw = ldt / 2 + 1, bsw = r / 2 + 1;  // row strides in 32-bit words
  uint32_t* tl = mc_lds;                   // [MC_ROWS][tsw]
  uint32_t* bl = mc_lds + MC_ROWS * tsw;   // [MC_COLS][bsw]
  const int m0 = blockIdx.y * MC_ROWS, n0 = blockIdx.x * MC_COLS;
  const int tid = threadIdx.x;
  if (r > 0) {  // 16-byte global chunks: ldt and r are multiples of 8
    const int tc = ldt / 8, bc = r / 8;
    for (int q = tid; q < MC_ROWS * tc; q += 256) {
      const int row = q / tc, c = q % tc;
      const int m = min(m0 + row, M - 1);
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(t + (int64_t)m * ldt + c * 8);
      uint32_t* d = tl + row * tsw + c * 4;
      d[0] = v[0]; d[1] = v[1]; d[2] = v[2]; d[3] = v[3];
    }
    for (int q = tid; q < MC_COLS * bc; q += 256) {
      const int row = q / bc, c = q % bc;
      const int n = min(n0 + row, N - 1);
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(b + (int64_t)n * ldb + c * 8);
      uint32_t* d = bl + row * bsw + c * 4;
      d[0] = v[0]; d[1] = v[1]; d[2] = v[2]; d[3] = v[3];
    }
    __syncthreads();
  }
  const int rl = tid / 8, cq = tid % 8;  // row, column quad
  const int m = m0 + rl, nb = n0 + cq * 4;
  if (m >= M || nb >= N) return;
  const int64_t slice = (int64_t)M * N;
  const int64_t e = (int64_t)m * N + nb;
  const int nn = N - nb < 4 ? N - nb : 4;
  float v[4];
  if (nn == 4 && (N & 3) == 0) {
    // split order kept; four loads in flight at a time rather than one round trip per split
    const f32x4_t* pv = reinterpret_cast<const f32x4_t*>(part + e);
    const int64_t sv = slice / 4;
    f32x4_t a = pv[0];
    int q = 1;
    for (; q + 4 <= splits; q += 4) {
      const f32x4_t a0 = pv[q * sv], a1 = pv[(q + 1) * sv], a2 = pv[(q + 2) * sv], a3 = pv[(q + 3) * sv];
      a += a0; a += a1; a += a2; a += a3;
    }
    for (; q < splits; ++q) a += pv[q * sv];
    v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
  } else {
    for (int c = 0; c < 4; ++c) {
      v[c] = 0.f;
      if (c < nn)
        for (int q = 0; q < splits; ++q) v[c] += part[q * slice + e + c];
    }
  }
  if (r > 0) {
    const uint32_t* trow = tl + rl * tsw;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int n = nb + c;
      const int goff = ((n >= ge0) + (n >= ge1) + (n >= ge2)) * r;
      const uint32_t* tw = trow + goff / 2;
      const uint32_t* bw = bl + (cq * 4 + c) * bsw;
      float d = 0.f;
      for (int j = 0; j < r / 2; ++j) {
        const uint32_t tv = tw[j], bv = bw[j];
        d += bf16_bits_to_f32(tv & 0xffffu) * bf16_bits_to_f32(bv & 0xffffu);
        d += bf16_bits_to_f32(tv >> 16) * bf16_bits_to_f32(bv >> 16);
      }
      v[c] += d;
    }
  }
  uint16_t* dst = y + (int64_t)m * ldy + nb;
  if (nn == 4) {
    *reinterpret_cast<uint2*>(dst) = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  } else {
    for (int c = 0; c < nn; ++c) dst[c] = f32_to_bf16_bits(v[c]);
  }
}

hipError_t launch_medium(const LoraArgs& p, int splits) {
  const int64_t rt = p.r * p.groups;
  uint16_t* t = reinterpret_cast<uint16_t*>(p.ws);
  const size_t t_bytes = p.r > 0 ? rank_prepass_bytes(p.M, p.K, rt) : 0;
  float* part = reinterpret_cast<float*>(reinterpret_cast<char*>(p.ws) + ((t_bytes + 255) & ~(size_t)255));
  if (p.r > 0) {
    const hipError_t e = rank_prepass(p, t);
    if (e != hipSuccess) return e;
  }
  LoraArgs q = p;
  q.a = nullptr; q.lda = 0; q.b = nullptr; q.ldb = 0; q.r = 0; q.groups = 1; q.yscale = 1.f;
  q.y = part; q.ldy = p.N; q.K = p.K / splits;
  hipError_t e = launch_cfg<CfgSmall, kBF16, true, 0, false, false, true>(q, nullptr, 0, splits);
  if (e != hipSuccess) return e;
  const dim3 grid((unsigned)((p.N + MC_COLS - 1) / MC_COLS), (unsigned)((p.M + MC_ROWS - 1) / MC_ROWS));
  const size_t lds = p.r > 0 ? (size_t)(MC_ROWS * (rt / 2 + 1) + MC_COLS * (p.r / 2 + 1)) * 4 : 0;  // < 34 KB
  medium_combine_kernel<<<grid, dim3(256), lds, p.stream>>>(
      part, splits, (int)p.M, (int)p.N, t, (int)rt, reinterpret_cast<const uint16_t*>(p.b), p.ldb, (int)p.r,
      group_end(p, 0), group_end(p, 1), group_end(p, 2), reinterpret_cast<uint16_t*>(p.y), p.ldy);
  return hipGetLastError();
}
}  // namespace

// Workspace of the prefill path: the rank pre-pass region (r > 32, where prepass_rank may
// take it; any rank on the fp8 matrix-core path or on the medium-M split path, which take T
// from the pre-pass), then for
// an fp8 W the activation codes of the fp8 matrix-core path, or the medium path's partials.
// With the in-launch split-K form possible (which `r`, the ranks of all groups, does not
// decide) its records are covered as well.
size_t prefill_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, int w_dtype) {
  if (w_dtype == kFP8)
    return (r > 0 ? rank_prepass_bytes(M, K, r) : 0) + prefill_fp8_workspace_bytes(M, K, 2);
  size_t b = r > 32 ? rank_prepass_bytes(M, K, r) : 0;
  const int ms = medium_splits(M, N, K, r, w_dtype, true, false);
  if (ms > 0) {
    const size_t t_bytes = r > 0 ? ((rank_prepass_bytes(M, K, r) + 255) & ~(size_t)255) : 0;
    b = std::max(b, t_bytes + (size_t)ms * M * N * 4);
  }
  const int rs = red_splits(M, N, K, w_dtype, true, false);
  if (rs > 0) b = std::max(b, (size_t)(((M + 127) / 128) * ((N + 127) / 128) * rs) * red_record_bytes());
  // shared T: one rank block per group (r here is the groups' total rank)
  if (r > 0 && r <= 32 * kMaxGroups) b = std::max(b, shared_t_bytes(M, N, K));
  return b;
}

// Pre-pass: T = bf16(s * x . A^T) [M, r] into the workspace, by the prefill kernel run as a
// plain GEMM with A in the place of W (N = r) and s applied before rounding. With few row
// tiles (N = r is one or two tiles wide) K is split over grid rows into fp32 partials that
// a second kernel sums in split order, scales and rounds; the splits run on the four-buffer
// ring (one workgroup per CU, three K tiles in flight), whose partial sums are those of the
// two-buffer form (the same K tiles and k steps in the same order). A grouped launch runs
// one pre-pass over all groups' A blocks (N = groups * r).
hipError_t rank_prepass(const LoraArgs& p, uint16_t* t) {
  const int64_t rt = p.r * p.groups;
  LoraArgs q = p;
  q.w = p.a; q.ldw = p.lda; q.w_dtype = kBF16; q.w_scale = nullptr;
  q.a = nullptr; q.lda = 0; q.b = nullptr; q.ldb = 0; q.r = 0; q.groups = 1;
  q.wmap = RowMap{}; q.wrows = rt;
  q.N = rt; q.y = t; q.ldy = rt; q.yscale = p.scale;
  const int splits = rank_splits(p.M, p.K, rt);
  if (splits > 1) {
    float* part = reinterpret_cast<float*>(reinterpret_cast<char*>(t) + (((size_t)(p.M * rt * 2) + 255) & ~(size_t)255));
    q.y = part; q.K = p.K / splits;
    hipError_t e = launch_cfg<CfgDeep, kBF16, true, 0, false, false, true>(q, nullptr, 0, splits);
    if (e != hipSuccess) return e;
    const int64_t slice = p.M * rt;
    rank_reduce_kernel<<<dim3((unsigned)((slice / 8 + 255) / 256)), dim3(256), 0, p.stream>>>(part, splits, slice, p.scale, t);
    return hipGetLastError();
  }
  return launch_rank<kBF16, true>(q, nullptr, 0);
}

// Plain bf16 products over a long contiguous K (the weight gradients, csrc/lora_backward.hip):
// y' = yscale * x' . W'^T, x' [M, K], W' [N, K]. The split count (a power of two, each part
// at least kMinSplitTiles K tiles, dividing the nk K tiles when `divides`): 1 when a tile
// configuration fills the CUs on its own, else K cut into equal parts over 128 x 128 tiles,
// fp32 partials. Scored by the fraction of the 256 CUs kept busy, 128 x 128 tiles at 0.78 of
// the larger tiles' loop rate and split partials at 0.95 for their fp32 round trip.
constexpr int kMaxProductSplits = 32;
int product_splits(int64_t M, int64_t N, int64_t nk, bool divides) {
  const int64_t tb = ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t ts = ((M + 127) / 128) * ((N + 127) / 128);
  double best = wave_efficiency(tb);
  if (0.78 * wave_efficiency(ts) > best) best = 0.78 * wave_efficiency(ts);
  int pick = 1;
  for (int s = 2; s <= kMaxProductSplits && s <= nk / kMinSplitTiles; s *= 2) {
    if (divides && nk % s != 0) break;
    const double sc = 0.78 * 0.95 * wave_efficiency(ts * s);
    if (sc > best + 1e-9) {
      best = sc;
      pick = s;
    }
  }
  return pick;
}

// part == nullptr (splits 1): bf16 y' (p.y, p.ldy) over the whole K by the tile choice of
// the forward, p.yscale applied; else unscaled fp32 partials [splits][M][N] into `part`, p.K
// being one part's length (the reduce applies the scale).
hipError_t launch_product(const LoraArgs& p, float* part, int splits) {
  LoraArgs q = p;
  q.w_dtype = kBF16; q.w_scale = nullptr; q.a = nullptr; q.lda = 0; q.b = nullptr; q.ldb = 0; q.r = 0;
  q.groups = 1; q.gather = nullptr; q.gather_rows = 0; q.wmap = RowMap{}; q.wrows = q.N;
  if (part == nullptr) return launch_rank<kBF16, true>(q, nullptr, 0);
  q.y = part; q.ldy = q.N;
  return launch_cfg<CfgSmall, kBF16, true, 0, false, false, true>(q, nullptr, 0, splits);
}

// Token-major products (the weight gradients): x' from p.x [tokens][M] (row stride ldx),
// W' from p.w [tokens][N] (ldw), bf16, M and N multiples of 8, 16-byte aligned rows;
// `tokens` rows in all, p.K per split (a multiple of BK; every split starts below `tokens`).
// part == nullptr (splits 1): bf16 y' (p.y, p.ldy, p.yscale) over 256 x 256 tiles when they
// fill the CUs, else 128 x 128; otherwise unscaled fp32 partials [splits][M][N] over 128 x 128.
hipError_t launch_product_tn(const LoraArgs& p, int64_t tokens, float* part, int splits) {
  LoraArgs q = p;
  q.w_dtype = kBF16; q.w_scale = nullptr; q.a = nullptr; q.lda = 0; q.b = nullptr; q.ldb = 0; q.r = 0;
  q.groups = 1; q.gather = nullptr; q.gather_rows = tokens; q.wmap = RowMap{}; q.wrows = q.N;
  if (part == nullptr) {
    const int64_t tb = ((q.M + 255) / 256) * ((q.N + 255) / 256);
    if (tb >= 192) return launch_cfg<CfgBig, kBF16, true, 0, false, false, false, true>(q, nullptr, 0);
    return launch_cfg<CfgSmall, kBF16, true, 0, false, false, false, true>(q, nullptr, 0);
  }
  q.y = part; q.ldy = q.N;
  return launch_cfg<CfgSmall, kBF16, true, 0, false, false, true, true>(q, nullptr, 0, splits);
}

int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int v = cus[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// The form, tile and splits a prefill call takes; launch_prefill follows it.
PrefillPlan plan_prefill(const LoraArgs& p) {
  PrefillPlan pl;
  pl.form = WSL_PATH_PREFILL;
  const bool has_w = p.w != nullptr;
  const int64_t rt = p.r * p.groups;
  const int64_t tiles128 = ((p.M + 127) / 128) * ((p.N + 127) / 128);
  if (p.gather != nullptr) {
    // factorized embedding: gathered x rows, bf16 base, no LoRA term
    const TilePick t = pick_tiles(p, kBF16, true, 0, false, true);
    pl.tile_m = tile_rows(t.tile);
    pl.tile_n = tile_cols(t.tile);
  } else if (has_w && p.w_dtype == kFP8 && fp8_matrix_cores(p)) {
    pl.form = WSL_PATH_PREFILL_FP8;
    pl.prepass = p.r > 0;
    pl.tile_m = pl.tile_n = 256;
  } else {
    // The in-launch split-K form runs 128 x 128 tiles that compute their group's T, so every
    // group end must fall on a tile boundary.
    const int rs = (has_w && p.w_dtype == kBF16 && p.r <= RIN && p.red_cnt != nullptr && groups_fit(p, 128))
                       ? red_splits(p.M, p.N, p.K, p.w_dtype, true, false)
                       : 0;
    const int ms = (rs == 0 && has_w && p.w_dtype == kBF16) ? medium_splits(p.M, p.N, p.K, rt, p.w_dtype, true, false)
                                                             : 0;
    if (rs > 0) {
      pl.form = WSL_PATH_PREFILL_SPLITK;
      pl.tile_m = pl.tile_n = 128;
      pl.rank_blocks = p.r == 0 ? 0 : p.r <= 32 ? 1 : 2;
      pl.splits = rs;
      pl.workgroups = tiles128 * rs;
      return pl;
    }
    if (ms > 0) {
      pl.form = WSL_PATH_PREFILL_MEDIUM;
      pl.tile_m = pl.tile_n = 128;
      pl.prepass = p.r > 0;
      pl.splits = ms;
      pl.workgroups = tiles128 * ms;
      return pl;
    }
    pl.prepass = p.r > 0 && prepass_rank(p);
    pl.rank_blocks = rank_blocks_of(p);
    const TilePick t = pick_tiles(p, has_w ? (int)p.w_dtype : kBF16, has_w, pl.rank_blocks, pl.prepass, false);
    pl.tile_m = tile_rows(t.tile);
    pl.tile_n = tile_cols(t.tile);
    pl.strips = t.strips;
    pl.shared_t = has_w && p.w_dtype == kBF16 && pl.rank_blocks == 1 && !pl.prepass && t.strips <= 1 &&
                  (t.tile == Tile::kBig || t.tile == Tile::kTall) && shared_t_rbgs(p, pl.tile_m, pl.tile_n) > 0;
  }
  pl.workgroups = ((p.M + pl.tile_m - 1) / pl.tile_m) * ((p.N + pl.tile_n - 1) / pl.tile_n) / pl.strips;
  return pl;
}

// ---- The input gradient with W read where it lies (the WT form) ----
// q is the forward-shaped problem of dX = dY . W + s (dY . B) . A for a linear with W [N, K]:
// x = dY [M, K'] (K' = N, the reduction), w = W with ldw its row stride (W'[n][k] =
// w[k * ldw + n]; N' = K output columns), a = B^T [r, K'], b = A^T [N', r], y = dX.
bool prefill_wt_supported(const LoraArgs& q) {
  if (q.groups != 1 || q.wmap.P != 0 || q.w == nullptr || q.gather != nullptr) return false;
  if (q.w_dtype == kFP8) {
    if (q.w_scale == nullptr || q.N % 16 != 0) return false;  // 16-byte chunks of e4m3 columns
  } else if (q.w_dtype != kBF16) {
    return false;
  }
  return q.M >= 1 && q.N % 8 == 0 && q.r <= WSL_MAX_RANK && prefill_supported(q);
}

namespace {
template <int WDT>
hipError_t launch_wt_rank(const LoraArgs& q, const uint16_t* tg, int64_t ldt) {
  if (tg != nullptr) return launch_variant<WDT, true, 0, true, false, true>(q, tg, ldt);
  if (q.r == 0) return launch_variant<WDT, true, 0, false, false, true>(q, nullptr, 0);
  if (q.r <= 32) return launch_variant<WDT, true, 1, false, false, true>(q, nullptr, 0);
  return launch_variant<WDT, true, 2, false, false, true>(q, nullptr, 0);
}
}  // namespace

// The forward's tile forms (tiles by how they fill the CUs, persistent strips, the three-
// and four-buffer rings), without the 192-wide tile (the token-major W' tile needs whole
// 128-column chunks). Ranks above 64 take T = s dY . B from the rank pre-pass in the
// workspace. An fp8 W is decoded through registers with each row's scale (bf16(code *
// scale), the values of the dequantised W) into the same token-major tiles (two-buffer
// ring, no strips).
hipError_t launch_prefill_wt(const LoraArgs& q_in) {
  LoraArgs q = q_in;
  q.gather_rows = q.K;  // every reduction row of W' is in range: no clamping in its fills
  const uint16_t* tg = nullptr;
  int64_t ldt = 0;
  // T from the pre-pass above RIN, and for ranks 33-64 where it frees a tile wider than
  // 128 x 128 (as the forward's prepass_rank)
  bool pre = q.r > RIN;
  if (!pre && q.r > 32) {
    const Tile t = pick_tiles(q, (int)q.w_dtype, true, 0, true, false, true).tile;
    pre = t != Tile::kSmall && t != Tile::kDeep;
  }
  if (pre) {
    uint16_t* t = reinterpret_cast<uint16_t*>(q.ws);
    const hipError_t e = rank_prepass(q, t);
    if (e != hipSuccess) return e;
    tg = t;
    ldt = q.r;
  }
  if (q.w_dtype == kFP8) return launch_wt_rank<kFP8>(q, tg, ldt);
  return launch_wt_rank<kBF16>(q, tg, ldt);
}

hipError_t launch_prefill(const LoraArgs& p) {
  if (p.gather != nullptr) {
    // factorized embedding: gathered x rows, bf16 base, no LoRA term
    return launch_variant<kBF16, true, 0, false, true>(p, nullptr, 0);
  }
  const bool has_w = p.w != nullptr;
  const int64_t rt = p.r * p.groups;
  uint16_t* t = reinterpret_cast<uint16_t*>(p.ws);
  const PrefillPlan pl = plan_prefill(p);
  if (pl.form == WSL_PATH_PREFILL_FP8) {
    if (p.r > 0) {
      const hipError_t e = rank_prepass(p, t);
      if (e != hipSuccess) return e;
    }
    char* codes = reinterpret_cast<char*>(p.ws) + (p.r > 0 ? rank_prepass_bytes(p.M, p.K, rt) : 0);
    return launch_prefill_fp8(p, p.r > 0 ? t : nullptr, rt, codes, p.fp8_terms);
  }
  if (pl.form == WSL_PATH_PREFILL_SPLITK) return launch_red(p, pl.splits);
  if (pl.form == WSL_PATH_PREFILL_MEDIUM) return launch_medium(p, pl.splits);
  const uint16_t* tg = nullptr;
  int64_t ldt = 0;
  if (pl.prepass) {
    const hipError_t e = rank_prepass(p, t);
    if (e != hipSuccess) return e;
    tg = t;
    ldt = rt;
  }
  if (has_w && p.w_dtype == kFP8) return launch_rank<kFP8, true>(p, tg, ldt);
  if (has_w) return launch_rank<kBF16, true>(p, tg, ldt);
  return launch_rank<kBF16, false>(p, tg, ldt);
}

}  // namespace wsl

#ifdef WSL_STAMPS
// Instrumented builds only: copies the first `recs` phase-stamp records (8 words each) to
// host memory, then clears them on the device. Returns 0 or a HIP error code.
extern "C" int wsl_prefill_stamps(unsigned long long* host, size_t recs) {
  if (recs > (size_t)wsl::kStampRecs) recs = wsl::kStampRecs;
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpyFromSymbol(host, HIP_SYMBOL(wsl::g_prefill_stamps), recs * 8 * sizeof(unsigned long long));
  static unsigned long long zeros[wsl::kStampRecs * 8];
  if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(wsl::g_prefill_stamps), zeros, sizeof(zeros));
  return (int)e;
}
#endif
