// Decode-step kernels of the weight-shared Qwen3 harness for gfx950: the work between
// the fused LoRA projections of one token step, each as one launch.
//
//   rmsnorm_kernel        h = x (+ residual, rounded to bf16); out = bf16(h * rsqrt(mean(h^2)
//                         + eps) * w). One workgroup per row.
//   qk_rope_kernel        per head of the step's q|k|v row: RMSNorm over head_dim (q, k),
//                         rotary embedding at the step's position, q written out, k and v
//                         written into the KV cache at that position. One wave per head.
//   attention_step        the q/k norm + RoPE + cache write of one step fused with its
//                         attention: every chunk workgroup normalises and rotates its own
//                         query heads; the chunk holding `pos` also the step's k (and v),
//                         writes them into the cache and uses them from LDS; the partial
//                         records are merged by the last chunk workgroup of each (sequence,
//                         kv head) to arrive (agent-scope atomics; arrival counters reset by
//                         that workgroup), so the whole step is one launch.
//   attention_partial     GQA attention of one query token against positions 0..pos of the
//   attention_combine     cache, split over the cache length: a workgroup takes 64 positions
//                         of one (sequence, kv head), 16-lane groups per position with all
//                         loads in flight at once, online softmax, groups combined through
//                         LDS into a partial (max, sum, weighted V); a second launch merges
//                         the partials of each (sequence, kv head).
//   swiglu_kernel         out = bf16(silu(g) * u) from the gate|up projection output.
//   argmax_kernel         greedy token: index of the largest logit of a row (first index on
//                         ties, NaN counted as largest, as torch.argmax). One workgroup per row.
//
// Arithmetic is fp32 with one rounding to bf16 per output (the torch ops they replace
// round after every op). Reference semantics: RMSNorm torchtitan/models/llama3/model/
// model.py (nn.RMSNorm in Qwen3 blocks, torchtitan/experiments/qwen3/model/model.py:
// 195-198, 296-314), RoPE :20-36,73-90, GQA attention :167-218, SwiGLU :250-251.
#include "../../include/wsl_decode.h"
#include "wsl_common.h"

namespace wsl {
namespace {

__device__ __forceinline__ float bf(uint16_t h) { return bf16_bits_to_f32(h); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// --------------------------------------------------------------------- RMSNorm
constexpr int RN_T = 256;     // threads per row
constexpr int RN_MAXC = 4;    // 16-byte chunks per thread: dim <= 256 * 8 * 4 = 8192

__global__ void __launch_bounds__(RN_T) rmsnorm_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                      const uint16_t* __restrict__ res, int64_t ldr,
                                                      const uint16_t* __restrict__ w, float eps,
                                                      uint16_t* __restrict__ out, int64_t ldo,
                                                      uint16_t* __restrict__ hout, int64_t ldh, int dim) {
  __shared__ float part[RN_T / 64];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int nch = dim >> 3;
  float h[RN_MAXC][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < RN_MAXC; ++c) {
    const int ch = tid + c * RN_T;
    if (ch < nch) {
      const u32x4_t xv = ld_global_16(x + (int64_t)row * ldx + ch * 8);
      u32x4_t rv = zero_u32x4();
      if (res != nullptr) rv = ld_global_16(res + (int64_t)row * ldr + ch * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float v = bf(xv[e >> 1] >> ((e & 1) * 16) & 0xffffu);
        if (res != nullptr) v = bf(f32_to_bf16_bits(v + bf(rv[e >> 1] >> ((e & 1) * 16) & 0xffffu)));
        h[c][e] = v;
        ss += v * v;
      }
      if (hout != nullptr) {
        u32x4_t hv;
#pragma unroll
        for (int q = 0; q < 4; ++q) hv[q] = pack_bf16x2(h[c][2 * q], h[c][2 * q + 1]);
        *reinterpret_cast<u32x4_t*>(hout + (int64_t)row * ldh + ch * 8) = hv;
      }
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < RN_T / 64; ++i) tot += part[i];
  const float inv = rsqrtf(tot / (float)dim + eps);
#pragma unroll
  for (int c = 0; c < RN_MAXC; ++c) {
    const int ch = tid + c * RN_T;
    if (ch < nch) {
      const u32x4_t wv = ld_global_16(w + ch * 8);
      u32x4_t ov;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        ov[q] = pack_bf16x2(h[c][2 * q] * inv * bf(wv[q] & 0xffffu), h[c][2 * q + 1] * inv * bf(wv[q] >> 16));
      *reinterpret_cast<u32x4_t*>(out + (int64_t)row * ldo + ch * 8) = ov;
    }
  }
}

// --------------------------------------------------------------------- q/k norm + RoPE + cache
// Lane l of a head's wave holds elements l + 64c, c < C (head_dim = 64 C). The rotation
// pairs element j with j + hd/2: the same lane's chunk c + C/2 when C >= 2, lane l ^ 32
// when C == 1.
template <int C>
__global__ void __launch_bounds__(256) qk_rope_kernel(const uint16_t* __restrict__ qkv, int64_t ldq, int batch,
                                                     int nh, int nkv, const uint16_t* __restrict__ qw,
                                                     const uint16_t* __restrict__ kw, float eps,
                                                     const float* __restrict__ rope, const int64_t* __restrict__ posp,
                                                     uint16_t* __restrict__ qout, uint16_t* __restrict__ kc,
                                                     uint16_t* __restrict__ vc, int cache_len) {
  constexpr int HD = 64 * C;
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);  // (sequence, head) of this wave
  const int heads = nh + nkv;
  if (gw >= batch * heads) return;
  const int b = gw / heads, hh = gw % heads;
  const bool is_q = hh < nh;
  const int64_t pos = *posp;
  if (pos < 0 || pos >= cache_len) {  // no rope row or cache slot: NaN q, nothing written
    if (is_q) {
      uint16_t* dst = qout + ((int64_t)b * nh + hh) * HD;
#pragma unroll
      for (int c = 0; c < C; ++c) dst[lane + 64 * c] = 0x7fc0;
    }
    return;
  }
  const uint16_t* src = qkv + (int64_t)b * ldq + (int64_t)hh * HD;
  const uint16_t* nw = is_q ? qw : kw;
  float v[C];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    v[c] = bf(src[lane + 64 * c]);
    ss += v[c] * v[c];
  }
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / (float)HD + eps);
  float n[C];
#pragma unroll
  for (int c = 0; c < C; ++c) n[c] = v[c] * inv * bf(nw[lane + 64 * c]);
  // rope table row `pos`: cos in [0, HD), sin in [HD, 2 HD)
  const float* rc = rope + pos * 2 * HD;
  float o[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int j = lane + 64 * c;
    float partner;
    if constexpr (C == 1) {
      partner = __shfl_xor(n[0], 32, 64);
    } else {
      partner = n[(c + C / 2) % C];
    }
    const float rot = (j < HD / 2) ? -partner : partner;  // rotate_half
    o[c] = n[c] * rc[j] + rot * rc[HD + j];
  }
  if (is_q) {
    uint16_t* dst = qout + ((int64_t)b * nh + hh) * HD;
#pragma unroll
    for (int c = 0; c < C; ++c) dst[lane + 64 * c] = f32_to_bf16_bits(o[c]);
  } else {
    const int kh = hh - nh;
    const int64_t base = (((int64_t)b * nkv + kh) * cache_len + pos) * HD;
    const uint16_t* vsrc = qkv + (int64_t)b * ldq + (int64_t)(nh + nkv + kh) * HD;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      kc[base + lane + 64 * c] = f32_to_bf16_bits(o[c]);
      vc[base + lane + 64 * c] = vsrc[lane + 64 * c];
    }
  }
}

// --------------------------------------------------------------------- decode attention
constexpr int AT_T = 256;              // 4 waves = 16 groups of 16 lanes
constexpr int AT_G = AT_T / 16;
constexpr int AT_CH = 64;              // cache positions per workgroup
constexpr int AT_U = AT_CH / AT_G;     // positions per group, all in flight
constexpr int AT_B = 8;                // record loads a thread keeps in flight in the merge
// Arrival counters: a fixed 64 KB region at the start of the workspace, which nothing
// else writes (the records follow it), so counters stay zero between calls of any shape.
// A pair's counter is on its own 128-byte line up to 512 pairs, packed closer beyond.
constexpr size_t AT_CREGION = 65536;
constexpr int64_t AT_MAX_PAIRS = (int64_t)(AT_CREGION / 4);
int at_cstride(int64_t pairs) {
  return pairs <= 512 ? 32 : (int)(AT_MAX_PAIRS / pairs);
}

// EPL (4 or 8) consecutive bf16 of a row as one 8- or 16-byte load.
template <int EPL> struct Vec;
template <> struct Vec<8> {
  u32x4_t v;
  __device__ __forceinline__ void load(const uint16_t* p) { v = ld_global_16(p); }
  __device__ __forceinline__ void load_lds(const uint16_t* p) { v = *reinterpret_cast<const u32x4_t*>(p); }
  __device__ __forceinline__ float at(int e) const { return bf((v[e >> 1] >> ((e & 1) * 16)) & 0xffffu); }
};
template <> struct Vec<4> {
  uint2 v;
  __device__ __forceinline__ void load(const uint16_t* p) { v = *reinterpret_cast<const uint2*>(p); }
  __device__ __forceinline__ void load_lds(const uint16_t* p) { v = *reinterpret_cast<const uint2*>(p); }
  __device__ __forceinline__ float at(int e) const {
    const uint32_t w = (e >> 1) ? v.y : v.x;
    return bf((w >> ((e & 1) * 16)) & 0xffffu);
  }
};

// Partial record of one (pair, chunk): per head the running max, the sum of exp and the
// exp-weighted V sum, [REP][HD + 2] floats.
template <int EPL, int REP>
__global__ void __launch_bounds__(AT_T) attention_partial(const uint16_t* __restrict__ q,
                                                         const uint16_t* __restrict__ kc,
                                                         const uint16_t* __restrict__ vc, int nh, int nkv,
                                                         int cache_len, int nchunk, const int64_t* __restrict__ posp,
                                                         float scale, float* __restrict__ part) {
  constexpr int HD = 16 * EPL;
  __shared__ float s_m[AT_G * REP], s_l[AT_G * REP];
  __shared__ float s_acc[AT_G * REP * HD];
  const int pair = blockIdx.x / nchunk, chunk = blockIdx.x % nchunk;
  const int64_t pos = *posp;
  if (pos < 0 || pos >= cache_len) return;  // the combine writes NaN
  const int L = (int)pos + 1;
  const int t0 = chunk * AT_CH;
  if (t0 >= L) return;  // the combine reads only the chunks below L
  const int b = pair / nkv, kvh = pair % nkv;
  const int tid = threadIdx.x;
  const int g = tid >> 4, l16 = tid & 15;
  float qv[REP][EPL];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    const uint16_t* qr = q + ((int64_t)b * nh + kvh * REP + h) * HD + l16 * EPL;
#pragma unroll
    for (int e = 0; e < EPL; ++e) qv[h][e] = bf(qr[e]) * scale;
  }
  const uint16_t* kbase = kc + (int64_t)pair * cache_len * HD + l16 * EPL;
  const uint16_t* vbase = vc + (int64_t)pair * cache_len * HD + l16 * EPL;
  Vec<EPL> kv[AT_U], vv[AT_U];
#pragma unroll
  for (int u = 0; u < AT_U; ++u) {
    const int t = min(t0 + g + u * AT_G, L - 1);
    kv[u].load(kbase + (int64_t)t * HD);
    vv[u].load(vbase + (int64_t)t * HD);
  }
  float m[REP], lsum[REP], acc[REP][EPL];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    m[h] = -INFINITY;
    lsum[h] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[h][e] = 0.f;
  }
#pragma unroll
  for (int u = 0; u < AT_U; ++u) {
    if (t0 + g + u * AT_G >= L) break;
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      float sc = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) sc += qv[h][e] * kv[u].at(e);
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) sc += __shfl_xor(sc, o, 16);
      const float mn = fmaxf(m[h], sc);
      const float corr = __expf(m[h] - mn);
      const float p = __expf(sc - mn);
      lsum[h] = lsum[h] * corr + p;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[h][e] = acc[h][e] * corr + p * vv[u].at(e);
      m[h] = mn;
    }
  }
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    if (l16 == 0) {
      s_m[g * REP + h] = m[h];
      s_l[g * REP + h] = lsum[h];
    }
#pragma unroll
    for (int e = 0; e < EPL; ++e) s_acc[(g * REP + h) * HD + l16 * EPL + e] = acc[h][e];
  }
  __syncthreads();
  float* rec = part + (int64_t)blockIdx.x * REP * (HD + 2);
  for (int q2 = tid; q2 < REP * HD; q2 += AT_T) {
    const int h = q2 / HD, d = q2 % HD;
    float mx = -INFINITY;
    for (int gg = 0; gg < AT_G; ++gg) mx = fmaxf(mx, s_m[gg * REP + h]);
    float num = 0.f, den = 0.f;
    for (int gg = 0; gg < AT_G; ++gg) {
      const float mg = s_m[gg * REP + h];
      if (mg == -INFINITY) continue;  // a group that saw no position
      const float f = __expf(mg - mx);
      num += f * s_acc[(gg * REP + h) * HD + d];
      den += f * s_l[gg * REP + h];
    }
    rec[h * (HD + 2) + d] = num;
    if (d == 0) {
      rec[h * (HD + 2) + HD] = mx;
      rec[h * (HD + 2) + HD + 1] = den;
    }
  }
}

// One workgroup per (sequence, kv head), one thread per (head, element): merges the
// partial records of the chunks below L.
template <int HD, int REP>
__global__ void __launch_bounds__(1024) attention_combine(const float* __restrict__ part, int nh, int nkv,
                                                         int cache_len, int nchunk, const int64_t* __restrict__ posp,
                                                         uint16_t* __restrict__ out) {
  const int pair = blockIdx.x;
  const int b = pair / nkv, kvh = pair % nkv;
  const int tid = threadIdx.x;
  if (tid >= REP * HD) return;
  const int h = tid / HD, d = tid % HD;
  const int64_t pos = *posp;
  if (pos < 0 || pos >= cache_len) {  // past the cache: no records were written
    out[((int64_t)b * nh + kvh * REP + h) * HD + d] = 0x7fc0;
    return;
  }
  const int L = (int)pos + 1;
  const int nc = min(nchunk, (L + AT_CH - 1) / AT_CH);
  const float* rec = part + (int64_t)pair * nchunk * REP * (HD + 2) + h * (HD + 2);
  float mx = -INFINITY;
  for (int c = 0; c < nc; ++c) mx = fmaxf(mx, rec[(int64_t)c * REP * (HD + 2) + HD]);
  float num = 0.f, den = 0.f;
  for (int c = 0; c < nc; ++c) {
    const float* rc = rec + (int64_t)c * REP * (HD + 2);
    const float f = __expf(rc[HD] - mx);
    num += f * rc[d];
    den += f * rc[HD + 1];
  }
  out[((int64_t)b * nh + kvh * REP + h) * HD + d] = f32_to_bf16_bits(num / den);
}

// --------------------------------------------------------------------- SwiGLU
__global__ void __launch_bounds__(256) swiglu_kernel(const uint16_t* __restrict__ gu, int64_t ld, int ffn,
                                                    uint16_t* __restrict__ out, int64_t ldo) {
  const int row = blockIdx.y;
  const int ch = blockIdx.x * 256 + threadIdx.x;  // 8-element chunk
  if (ch * 8 >= ffn) return;
  const u32x4_t gv = ld_global_16(gu + (int64_t)row * ld + ch * 8);
  const u32x4_t uv = ld_global_16(gu + (int64_t)row * ld + ffn + ch * 8);
  u32x4_t ov;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float r[2];
#pragma unroll
    for (int hlf = 0; hlf < 2; ++hlf) {
      const float gg = bf((gv[q] >> (16 * hlf)) & 0xffffu);
      const float uu = bf((uv[q] >> (16 * hlf)) & 0xffffu);
      r[hlf] = gg / (1.f + __expf(-gg)) * uu;
    }
    ov[q] = pack_bf16x2(r[0], r[1]);
  }
  *reinterpret_cast<u32x4_t*>(out + (int64_t)row * ldo + ch * 8) = ov;
}

// --------------------------------------------------------------------- argmax
constexpr int AM_T = 1024;
constexpr int AM_U = 8;     // 16-byte loads a thread keeps in flight

// (v, i) beats (w, j): NaN above every number, then the larger value, then the smaller index.
__device__ __forceinline__ bool am_better(float v, int64_t i, float w, int64_t j) {
  const bool vn = v != v, wn = w != w;
  if (vn != wn) return vn;
  if (!vn && v != w) return v > w;
  return i < j;
}

__global__ void __launch_bounds__(AM_T) argmax_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t n,
                                                     int vec, int64_t* __restrict__ out) {
  __shared__ float sv[AM_T / 64];
  __shared__ int64_t si[AM_T / 64];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* xr = x + (int64_t)row * ldx;
  float bv = -INFINITY;
  int64_t bi = INT64_MAX;
  const int64_t nch = vec ? (n >> 3) : 0;  // 16-byte chunks (aligned rows only), then a scalar tail
  int64_t c = tid;
  for (; c + (AM_U - 1) * AM_T < nch; c += AM_U * AM_T) {  // AM_U loads in flight per thread
    u32x4_t v[AM_U];
#pragma unroll
    for (int u = 0; u < AM_U; ++u) v[u] = ld_global_16(xr + (c + u * AM_T) * 8);
#pragma unroll
    for (int u = 0; u < AM_U; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = bf((v[u][e >> 1] >> ((e & 1) * 16)) & 0xffffu);
        const int64_t k = (c + u * AM_T) * 8 + e;
        if (am_better(f, k, bv, bi)) { bv = f; bi = k; }
      }
  }
  for (; c < nch; c += AM_T) {
    const u32x4_t v = ld_global_16(xr + c * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = bf((v[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
      if (am_better(f, c * 8 + e, bv, bi)) { bv = f; bi = c * 8 + e; }
    }
  }
  for (int64_t k = nch * 8 + tid; k < n; k += AM_T) {  // tail
    const float f = bf(xr[k]);
    if (am_better(f, k, bv, bi)) { bv = f; bi = k; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int64_t oi = __shfl_xor(bi, o, 64);
    if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if ((tid & 63) == 0) { sv[tid >> 6] = bv; si[tid >> 6] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < AM_T / 64; ++w)
      if (am_better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
    out[row] = bi;
  }
}

// Split argmax: a row's chunks are reduced by separate workgroups and merged with a 64-bit
// atomic max on a key that orders (value, then the lower index) as am_better does: the
// value's order-preserving bits (NaN above everything, -0 folded into +0) over the
// complemented index. The last chunk of a row (arrival counter) takes the key with an
// atomic exchange, writes the index and returns the counter to zero. The atomics are
// relaxed (each chunk waits for its maximum to be performed before it arrives, and the key
// is read by an atomic at the same scope): a release/acquire pair would add an L2
// write-back and invalidate to every chunk. Workspace: per row, the key and the counter on
// lines of their own (AMS_ROW bytes).
constexpr int AMS_T = 256;
constexpr int64_t AMS_CHUNK = 4096;  // elements per workgroup (at least)
constexpr int AMS_MAXS = 64;         // chunks per row (at most)
constexpr size_t AMS_ROW = 256;

__global__ void __launch_bounds__(AMS_T) argmax_split_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t n,
                                                            int vec, int nsplit, int64_t chunk,
                                                            char* __restrict__ ws, int64_t* __restrict__ out) {
  __shared__ float sv[AMS_T / 64];
  __shared__ int64_t si[AMS_T / 64];
  const int row = blockIdx.x / nsplit, sp = blockIdx.x % nsplit;
  const int tid = threadIdx.x;
  const uint16_t* xr = x + (int64_t)row * ldx;
  const int64_t k0 = sp * chunk, k1 = min(n, k0 + chunk);
  float bv = -INFINITY;
  int64_t bi = INT64_MAX;
  int64_t k = k0;
  if (vec) {  // chunk is a multiple of 8 and the rows are 16-byte aligned
    const int64_t c1 = k0 / 8 + (k1 - k0) / 8;
    for (int64_t c = k0 / 8 + tid; c < c1; c += AMS_T) {
      const u32x4_t v = ld_global_16(xr + c * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = bf((v[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
        if (am_better(f, c * 8 + e, bv, bi)) { bv = f; bi = c * 8 + e; }
      }
    }
    k = c1 * 8;
  }
  for (int64_t kk = k + tid; kk < k1; kk += AMS_T) {  // tail (or the whole chunk without vec)
    const float f = bf(xr[kk]);
    if (am_better(f, kk, bv, bi)) { bv = f; bi = kk; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int64_t oi = __shfl_xor(bi, o, 64);
    if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if ((tid & 63) == 0) { sv[tid >> 6] = bv; si[tid >> 6] = bi; }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < AMS_T / 64; ++w)
      if (am_better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
    uint64_t* key = reinterpret_cast<uint64_t*>(ws + (size_t)row * AMS_ROW);
    unsigned* cnt = reinterpret_cast<unsigned*>(ws + (size_t)row * AMS_ROW + 128);
    if (bi != INT64_MAX) __hip_atomic_fetch_max(key, am_key(bv, bi), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the maximum is performed before the arrival
    const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == (unsigned)(nsplit - 1)) {  // every chunk's key is in: take it, leaving zero
      out[row] = am_index(__hip_atomic_exchange(key, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ------------------------------------------------------------ fused step (norm + RoPE + attention)
__device__ __forceinline__ void st_agent_f(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent_f(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int EPL, int REP>
__global__ void __launch_bounds__(AT_T) attention_step(const uint16_t* __restrict__ qkv, int64_t ldq, int nh, int nkv,
                                                      const uint16_t* __restrict__ qw, const uint16_t* __restrict__ kw,
                                                      float eps, const float* __restrict__ rope,
                                                      const int64_t* __restrict__ posp, uint16_t* __restrict__ kc,
                                                      uint16_t* __restrict__ vc, int cache_len, int nchunk, float scale,
                                                      unsigned* __restrict__ cnt, int cstride, float* __restrict__ part,
                                                      uint16_t* __restrict__ out) {
  constexpr int HD = 16 * EPL;
  constexpr int C = HD / 64;  // elements per lane when one wave holds one head
  __shared__ float s_q[REP * HD];
  __shared__ uint16_t s_knew[HD], s_vnew[HD];
  __shared__ float s_m[AT_G * REP], s_l[AT_G * REP];
  __shared__ float s_acc[AT_G * REP * HD];
  __shared__ int s_last;
  const int pair = blockIdx.x / nchunk, chunk = blockIdx.x % nchunk;
  const int b = pair / nkv, kvh = pair % nkv;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t pos64 = *posp;
  if (pos64 < 0 || pos64 >= cache_len) {  // no rope row or cache slot: NaN out, nothing written
    if (chunk == 0)
      for (int q2 = tid; q2 < REP * HD; q2 += AT_T) out[((int64_t)b * nh + kvh * REP) * HD + q2] = 0x7fc0;
    return;
  }
  const int pos = (int)pos64;
  const int L = pos + 1;
  const int t0 = chunk * AT_CH;
  if (t0 >= L) return;  // no position here; the merge counts only the chunks below L
  const int g = tid >> 4, l16 = tid & 15;
  const bool owner = (pos / AT_CH) == chunk;
  const float* rc = rope + (int64_t)pos * 2 * HD;
  // K/V of this group's positions, issued first so their latency overlaps the q work below.
  // Position `pos` reads stale cache here; it is replaced from LDS after the barrier.
  const uint16_t* kbase = kc + (int64_t)pair * cache_len * HD + l16 * EPL;
  const uint16_t* vbase = vc + (int64_t)pair * cache_len * HD + l16 * EPL;
  Vec<EPL> kv[AT_U], vv[AT_U];
#pragma unroll
  for (int u = 0; u < AT_U; ++u) {
    const int t = min(t0 + g + u * AT_G, pos);
    kv[u].load(kbase + (int64_t)t * HD);
    vv[u].load(vbase + (int64_t)t * HD);
  }
  // q heads of this kv head (and, in the owner chunk, the step's k head): one wave each
  const int nheads = REP + (owner ? 1 : 0);
  for (int hh = wave; hh < nheads; hh += AT_T / 64) {
    const bool is_q = hh < REP;
    const int head = is_q ? kvh * REP + hh : nh + kvh;
    const uint16_t* src = qkv + (int64_t)b * ldq + (int64_t)head * HD;
    const uint16_t* nw = is_q ? qw : kw;
    float v[C], ss = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      v[c] = bf(src[lane + 64 * c]);
      ss += v[c] * v[c];
    }
    ss = wave_sum(ss);
    const float inv = rsqrtf(ss / (float)HD + eps);
    float n[C];
#pragma unroll
    for (int c = 0; c < C; ++c) n[c] = v[c] * inv * bf(nw[lane + 64 * c]);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int j = lane + 64 * c;
      float partner;
      if constexpr (C == 1) partner = __shfl_xor(n[0], 32, 64);
      else partner = n[(c + C / 2) % C];
      const float rot = (j < HD / 2) ? -partner : partner;  // rotate_half
      const float o = n[c] * rc[j] + rot * rc[HD + j];
      if (is_q) {
        s_q[hh * HD + j] = o * scale;
      } else {
        const int64_t at = ((int64_t)pair * cache_len + pos) * HD + j;
        const uint16_t kb = f32_to_bf16_bits(o);
        const uint16_t vb = qkv[(int64_t)b * ldq + (int64_t)(nh + nkv + kvh) * HD + j];
        s_knew[j] = kb;
        s_vnew[j] = vb;
        kc[at] = kb;
        vc[at] = vb;
      }
    }
  }
  __syncthreads();
  float qv[REP][EPL];
#pragma unroll
  for (int h = 0; h < REP; ++h)
#pragma unroll
    for (int e = 0; e < EPL; ++e) qv[h][e] = s_q[h * HD + l16 * EPL + e];
#pragma unroll
  for (int u = 0; u < AT_U; ++u) {
    if (min(t0 + g + u * AT_G, pos) == pos) {  // this step's k and v, from LDS
      kv[u].load_lds(s_knew + l16 * EPL);
      vv[u].load_lds(s_vnew + l16 * EPL);
    }
  }
  float m[REP], lsum[REP], acc[REP][EPL];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    m[h] = -INFINITY;
    lsum[h] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[h][e] = 0.f;
  }
#pragma unroll
  for (int u = 0; u < AT_U; ++u) {
    if (t0 + g + u * AT_G >= L) break;
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      float sc = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) sc += qv[h][e] * kv[u].at(e);
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) sc += __shfl_xor(sc, o, 16);
      const float mn = fmaxf(m[h], sc);
      const float corr = __expf(m[h] - mn);
      const float p = __expf(sc - mn);
      lsum[h] = lsum[h] * corr + p;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[h][e] = acc[h][e] * corr + p * vv[u].at(e);
      m[h] = mn;
    }
  }
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    if (l16 == 0) {
      s_m[g * REP + h] = m[h];
      s_l[g * REP + h] = lsum[h];
    }
#pragma unroll
    for (int e = 0; e < EPL; ++e) s_acc[(g * REP + h) * HD + l16 * EPL + e] = acc[h][e];
  }
  __syncthreads();
  // this chunk's record, published with agent-scope stores
  float* rec = part + (int64_t)blockIdx.x * REP * (HD + 2);
  for (int q2 = tid; q2 < REP * HD; q2 += AT_T) {
    const int h = q2 / HD, d = q2 % HD;
    float mx = -INFINITY;
    for (int gg = 0; gg < AT_G; ++gg) mx = fmaxf(mx, s_m[gg * REP + h]);
    float num = 0.f, den = 0.f;
    for (int gg = 0; gg < AT_G; ++gg) {
      const float mg = s_m[gg * REP + h];
      if (mg == -INFINITY) continue;
      const float f = __expf(mg - mx);
      num += f * s_acc[(gg * REP + h) * HD + d];
      den += f * s_l[gg * REP + h];
    }
    st_agent_f(rec + h * (HD + 2) + d, num);
    if (d == 0) {
      st_agent_f(rec + h * (HD + 2) + HD, mx);
      st_agent_f(rec + h * (HD + 2) + HD + 1, den);
    }
  }
  const int nc = (L + AT_CH - 1) / AT_CH;
  if (nc > 1) {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the record is out before the arrival
    __syncthreads();
    if (tid == 0) {
      unsigned* pc = cnt + pair * cstride;
      const unsigned old = __hip_atomic_fetch_add(pc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = old == (unsigned)(nc - 1);
      if (last) __hip_atomic_store(pc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
  } else {
    __builtin_amdgcn_s_waitcnt(0x0f70);
    __syncthreads();
  }
  // merge the records of every chunk of this pair (in chunk order): all loads issued at
  // once into LDS (the group buffers are free), then combined from there
  const float* base = part + (int64_t)pair * nchunk * REP * (HD + 2);
  constexpr int REC = REP * (HD + 2);
  constexpr int PASS = (AT_G * REP * HD) / REC;  // records staged per pass (>= 15)
  constexpr int NE = (REP * HD + AT_T - 1) / AT_T;
  float* s_rec = s_acc;  // the group buffers are free
  float rmx[NE], rnum[NE], rden[NE];
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    rmx[i] = -INFINITY;
    rnum[i] = 0.f;
    rden[i] = 0.f;
  }
  for (int c0 = 0; c0 < nc; c0 += PASS) {
    const int cn = min(PASS, nc - c0);
    __syncthreads();  // the previous pass is consumed
    // AT_B loads in flight per thread (clamped addresses: the loads are unconditional)
    const int nrec = cn * REC;
    for (int q0 = 0; q0 < nrec; q0 += AT_B * AT_T) {
      float v[AT_B];
#pragma unroll
      for (int u = 0; u < AT_B; ++u)
        v[u] = ld_agent_f(base + (int64_t)c0 * REC + min(q0 + u * AT_T + tid, nrec - 1));
#pragma unroll
      for (int u = 0; u < AT_B; ++u)
        if (q0 + u * AT_T + tid < nrec) s_rec[q0 + u * AT_T + tid] = v[u];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int q2 = tid + i * AT_T;
      if (q2 >= REP * HD) break;
      const int h = q2 / HD, d = q2 % HD;
      for (int c = 0; c < cn; ++c) {
        const float* r2 = s_rec + c * REC + h * (HD + 2);
        const float mn = fmaxf(rmx[i], r2[HD]);
        const float fo = __expf(rmx[i] - mn), fc = __expf(r2[HD] - mn);
        rnum[i] = rnum[i] * fo + r2[d] * fc;
        rden[i] = rden[i] * fo + r2[HD + 1] * fc;
        rmx[i] = mn;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    const int q2 = tid + i * AT_T;
    if (q2 >= REP * HD) break;
    const int h = q2 / HD, d = q2 % HD;
    out[((int64_t)b * nh + kvh * REP + h) * HD + d] = f32_to_bf16_bits(rnum[i] / rden[i]);
  }
}

template <int EPL, int R>
hipError_t launch_attention_r(int pairs, int nchunk, hipStream_t st, const uint16_t* q, const uint16_t* kc,
                              const uint16_t* vc, int nh, int nkv, int cache_len, const int64_t* pos, float scale,
                              float* part, uint16_t* out) {
  attention_partial<EPL, R><<<dim3((unsigned)(pairs * nchunk)), dim3(AT_T), 0, st>>>(q, kc, vc, nh, nkv, cache_len,
                                                                                   nchunk, pos, scale, part);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  attention_combine<16 * EPL, R><<<dim3((unsigned)pairs), dim3(1024), 0, st>>>(part, nh, nkv, cache_len, nchunk,
                                                                               pos, out);
  return hipGetLastError();
}

template <int EPL>
hipError_t launch_attention(int rep, int pairs, int nchunk, hipStream_t st, const uint16_t* q,
                            const uint16_t* kc, const uint16_t* vc, int nh, int nkv, int cache_len,
                            const int64_t* pos, float scale, float* part, uint16_t* out) {
  switch (rep) {
#define WSL_AT(R) \
  case R: return launch_attention_r<EPL, R>(pairs, nchunk, st, q, kc, vc, nh, nkv, cache_len, pos, scale, part, out);
    WSL_AT(1) WSL_AT(2) WSL_AT(4) WSL_AT(8)
#undef WSL_AT
    default: return hipErrorInvalidValue;
  }
}

}  // namespace
}  // namespace wsl

using namespace wsl;

namespace {
thread_local char g_derr[256] = {0};
int dfail(int code, const char* msg) {
  snprintf(g_derr, sizeof(g_derr), "%s", msg);
  return code;
}
}  // namespace

extern "C" {

const char* wsl_decode_last_error(void) { return g_derr; }

int wsl_rmsnorm_fwd(const void* x, int64_t ldx, const void* residual, int64_t ldr, const void* weight,
                    float eps, void* out, int64_t ldo, void* h_out, int64_t ldh, int64_t rows, int64_t dim,
                    void* stream) {
  g_derr[0] = 0;
  if (rows < 0 || dim < 8 || dim % 8 != 0 || dim > RN_T * 8 * RN_MAXC)
    return dfail(WSL_E_SHAPE, "rmsnorm: dim must be a multiple of 8 in [8, 8192], rows >= 0");
  if (rows == 0) return WSL_OK;
  if (x == nullptr || weight == nullptr || out == nullptr) return dfail(WSL_E_INVALID_ARG, "rmsnorm: null pointer");
  if (ldx < dim || ldo < dim || (residual != nullptr && ldr < dim) || (h_out != nullptr && ldh < dim))
    return dfail(WSL_E_SHAPE, "rmsnorm: leading dimension below dim");
  if (!a16(x) || !a16(weight) || !a16(out) || (residual != nullptr && !a16(residual)) ||
      (h_out != nullptr && !a16(h_out)) || ldx % 8 || ldo % 8 || (residual != nullptr && ldr % 8) ||
      (h_out != nullptr && ldh % 8))
    return dfail(WSL_E_ALIGN, "rmsnorm: pointers must be 16-byte aligned, leading dims multiples of 8");
  rmsnorm_kernel<<<dim3((unsigned)rows), dim3(RN_T), 0, reinterpret_cast<hipStream_t>(stream)>>>(
      (const uint16_t*)x, ldx, (const uint16_t*)residual, ldr, (const uint16_t*)weight, eps, (uint16_t*)out,
      ldo, (uint16_t*)h_out, ldh, (int)dim);
  return hipGetLastError() == hipSuccess ? WSL_OK : dfail(WSL_E_LAUNCH, "rmsnorm: launch failed");
}

int wsl_qk_norm_rope_fwd(const void* qkv, int64_t ldqkv, int64_t batch, int64_t n_heads, int64_t n_kv_heads,
                         int64_t head_dim, const void* q_norm_w, const void* k_norm_w, float eps,
                         const float* rope, const int64_t* pos, void* q_out, void* k_cache, void* v_cache,
                         int64_t cache_len, void* stream) {
  g_derr[0] = 0;
  if (batch < 0 || n_heads < 1 || n_kv_heads < 1 || cache_len < 1)
    return dfail(WSL_E_SHAPE, "qk_norm_rope: bad sizes");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return dfail(WSL_E_SHAPE, "qk_norm_rope: head_dim must be 64, 128 or 256");
  if (ldqkv < (n_heads + 2 * n_kv_heads) * head_dim) return dfail(WSL_E_SHAPE, "qk_norm_rope: ldqkv too small");
  if (batch == 0) return WSL_OK;
  if (!qkv || !q_norm_w || !k_norm_w || !rope || !pos || !q_out || !k_cache || !v_cache)
    return dfail(WSL_E_INVALID_ARG, "qk_norm_rope: null pointer");
  const int64_t waves = batch * (n_heads + n_kv_heads);
  dim3 grid((unsigned)((waves + 3) / 4));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define WSL_QK(CC)                                                                                             \
  qk_rope_kernel<CC><<<grid, dim3(256), 0, st>>>((const uint16_t*)qkv, ldqkv, (int)batch, (int)n_heads,     \
                                                 (int)n_kv_heads, (const uint16_t*)q_norm_w,                 \
                                                 (const uint16_t*)k_norm_w, eps, rope, pos, (uint16_t*)q_out, \
                                                 (uint16_t*)k_cache, (uint16_t*)v_cache, (int)cache_len)
  if (head_dim == 64) WSL_QK(1);
  else if (head_dim == 128) WSL_QK(2);
  else WSL_QK(4);
#undef WSL_QK
  return hipGetLastError() == hipSuccess ? WSL_OK : dfail(WSL_E_LAUNCH, "qk_norm_rope: launch failed");
}

size_t wsl_decode_attention_workspace_bytes(int64_t batch, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                             int64_t cache_len) {
  if (batch < 0 || n_heads < 1 || n_kv_heads < 1 || head_dim < 1 || cache_len < 1) return 0;
  const int64_t nchunk = (cache_len + AT_CH - 1) / AT_CH;
  return (size_t)(batch * n_heads * nchunk * (head_dim + 2) * 4);
}

int wsl_decode_attention_fwd(const void* q, const void* k_cache, const void* v_cache, int64_t batch,
                             int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t cache_len,
                             const int64_t* pos, float scale, void* out, void* workspace, size_t workspace_bytes,
                             void* stream) {
  g_derr[0] = 0;
  if (batch < 0 || n_kv_heads < 1 || n_heads % n_kv_heads != 0 || cache_len < 1)
    return dfail(WSL_E_SHAPE, "decode_attention: bad sizes");
  const int64_t rep = n_heads / n_kv_heads;
  if (rep != 1 && rep != 2 && rep != 4 && rep != 8)
    return dfail(WSL_E_SHAPE, "decode_attention: n_heads / n_kv_heads must be 1, 2, 4 or 8");
  if (head_dim != 64 && head_dim != 128) return dfail(WSL_E_SHAPE, "decode_attention: head_dim must be 64 or 128");
  if (batch == 0) return WSL_OK;
  if (!q || !k_cache || !v_cache || !pos || !out) return dfail(WSL_E_INVALID_ARG, "decode_attention: null pointer");
  const size_t need = wsl_decode_attention_workspace_bytes(batch, n_heads, n_kv_heads, head_dim, cache_len);
  if (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 15))
    return dfail(WSL_E_WORKSPACE, "decode_attention: workspace missing, too small or misaligned");
  const int pairs = (int)(batch * n_kv_heads);
  const int nchunk = (int)((cache_len + AT_CH - 1) / AT_CH);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e = head_dim == 64
                     ? launch_attention<4>((int)rep, pairs, nchunk, st, (const uint16_t*)q, (const uint16_t*)k_cache,
                                           (const uint16_t*)v_cache, (int)n_heads, (int)n_kv_heads, (int)cache_len,
                                           pos, scale, (float*)workspace, (uint16_t*)out)
                     : launch_attention<8>((int)rep, pairs, nchunk, st, (const uint16_t*)q, (const uint16_t*)k_cache,
                                           (const uint16_t*)v_cache, (int)n_heads, (int)n_kv_heads, (int)cache_len,
                                           pos, scale, (float*)workspace, (uint16_t*)out);
  return e == hipSuccess ? WSL_OK : dfail(WSL_E_LAUNCH, "decode_attention: launch failed");
}

size_t wsl_decode_attention_step_workspace_bytes(int64_t batch, int64_t n_heads, int64_t n_kv_heads,
                                                  int64_t head_dim, int64_t cache_len) {
  if (batch < 0 || n_heads < 1 || n_kv_heads < 1 || head_dim < 1 || cache_len < 1) return 0;
  const int64_t nchunk = (cache_len + AT_CH - 1) / AT_CH;
  return AT_CREGION + (size_t)(batch * n_heads * nchunk * (head_dim + 2) * 4);
}

int wsl_decode_attention_step_fwd(const void* qkv, int64_t ldqkv, int64_t batch, int64_t n_heads,
                                  int64_t n_kv_heads, int64_t head_dim, const void* q_norm_w, const void* k_norm_w,
                                  float eps, const float* rope, const int64_t* pos, void* k_cache, void* v_cache,
                                  int64_t cache_len, float scale, void* out, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  g_derr[0] = 0;
  if (batch < 0 || n_kv_heads < 1 || n_heads % n_kv_heads != 0 || cache_len < 1)
    return dfail(WSL_E_SHAPE, "decode_attention_step: bad sizes");
  const int64_t rep = n_heads / n_kv_heads;
  if (rep != 1 && rep != 2 && rep != 4)
    return dfail(WSL_E_SHAPE, "decode_attention_step: n_heads / n_kv_heads must be 1, 2 or 4");
  if (head_dim != 64 && head_dim != 128) return dfail(WSL_E_SHAPE, "decode_attention_step: head_dim must be 64 or 128");
  if (ldqkv < (n_heads + 2 * n_kv_heads) * head_dim) return dfail(WSL_E_SHAPE, "decode_attention_step: ldqkv too small");
  if (batch == 0) return WSL_OK;
  if (batch * n_kv_heads > AT_MAX_PAIRS)
    return dfail(WSL_E_SHAPE, "decode_attention_step: batch * n_kv_heads above 16384");
  if (!qkv || !q_norm_w || !k_norm_w || !rope || !pos || !k_cache || !v_cache || !out)
    return dfail(WSL_E_INVALID_ARG, "decode_attention_step: null pointer");
  const size_t need = wsl_decode_attention_step_workspace_bytes(batch, n_heads, n_kv_heads, head_dim, cache_len);
  if (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace & 255))
    return dfail(WSL_E_WORKSPACE, "decode_attention_step: workspace missing, too small or not 256-byte aligned");
  const int pairs = (int)(batch * n_kv_heads);
  const int nchunk = (int)((cache_len + AT_CH - 1) / AT_CH);
  unsigned* cnt = reinterpret_cast<unsigned*>(workspace);
  float* part = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + AT_CREGION);
  const int cstride = at_cstride(pairs);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((unsigned)(pairs * nchunk));
#define WSL_AS(E, R)                                                                                           \
  attention_step<E, R><<<grid, dim3(AT_T), 0, st>>>((const uint16_t*)qkv, ldqkv, (int)n_heads, (int)n_kv_heads, \
                                                    (const uint16_t*)q_norm_w, (const uint16_t*)k_norm_w, eps, rope, \
                                                    pos, (uint16_t*)k_cache, (uint16_t*)v_cache, (int)cache_len,     \
                                                    nchunk, scale, cnt, cstride, part, (uint16_t*)out)
  if (head_dim == 64) {
    if (rep == 1) WSL_AS(4, 1); else if (rep == 2) WSL_AS(4, 2); else WSL_AS(4, 4);
  } else {
    if (rep == 1) WSL_AS(8, 1); else if (rep == 2) WSL_AS(8, 2); else WSL_AS(8, 4);
  }
#undef WSL_AS
  return hipGetLastError() == hipSuccess ? WSL_OK : dfail(WSL_E_LAUNCH, "decode_attention_step: launch failed");
}

size_t wsl_argmax_rows_workspace_bytes(int64_t rows, int64_t n) {
  if (rows < 0 || n < 1) return 0;
  return (size_t)rows * AMS_ROW;
}

int wsl_argmax_rows_fwd(const void* x, int64_t ldx, int64_t rows, int64_t n, int64_t* out, void* workspace,
                        size_t workspace_bytes, void* stream) {
  g_derr[0] = 0;
  if (rows < 0 || n < 1 || ldx < n) return dfail(WSL_E_SHAPE, "argmax: bad sizes");
  if (rows == 0) return WSL_OK;
  if (!x || !out) return dfail(WSL_E_INVALID_ARG, "argmax: null pointer");
  if (((uintptr_t)x & 1) || ((uintptr_t)out & 7)) return dfail(WSL_E_ALIGN, "argmax: misaligned pointer");
  const int vec = (a16(x) && ldx % 8 == 0) ? 1 : 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (workspace == nullptr) {  // one workgroup per row
    argmax_kernel<<<dim3((unsigned)rows), dim3(AM_T), 0, st>>>((const uint16_t*)x, ldx, n, vec, out);
  } else {
    if (workspace_bytes < wsl_argmax_rows_workspace_bytes(rows, n) || ((uintptr_t)workspace & 255))
      return dfail(WSL_E_WORKSPACE, "argmax: workspace too small or not 256-byte aligned");
    if (n > (int64_t)0xffffffffLL) return dfail(WSL_E_SHAPE, "argmax: n above 2^32 - 1 with a workspace");
    int64_t chunk = (n + AMS_MAXS - 1) / AMS_MAXS;
    if (chunk < AMS_CHUNK) chunk = AMS_CHUNK;
    chunk = (chunk + 7) / 8 * 8;
    const int nsplit = (int)((n + chunk - 1) / chunk);
    if (rows * nsplit > (int64_t)INT32_MAX) return dfail(WSL_E_SHAPE, "argmax: too many rows");
    argmax_split_kernel<<<dim3((unsigned)(rows * nsplit)), dim3(AMS_T), 0, st>>>(
        (const uint16_t*)x, ldx, n, vec, nsplit, chunk, (char*)workspace, out);
  }
  return hipGetLastError() == hipSuccess ? WSL_OK : dfail(WSL_E_LAUNCH, "argmax: launch failed");
}

int wsl_swiglu_fwd(const void* gate_up, int64_t ld, int64_t rows, int64_t ffn, void* out, int64_t ldo,
                   void* stream) {
  g_derr[0] = 0;
  if (rows < 0 || ffn < 8 || ffn % 8 != 0 || ld < 2 * ffn || ldo < ffn) return dfail(WSL_E_SHAPE, "swiglu: bad sizes");
  if (rows == 0) return WSL_OK;
  if (!gate_up || !out) return dfail(WSL_E_INVALID_ARG, "swiglu: null pointer");
  if (!a16(gate_up) || !a16(out) || ld % 8 || ldo % 8) return dfail(WSL_E_ALIGN, "swiglu: 16-byte alignment required");
  dim3 grid((unsigned)((ffn / 8 + 255) / 256), (unsigned)rows);
  swiglu_kernel<<<grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream)>>>((const uint16_t*)gate_up, ld, (int)ffn,
                                                                               (uint16_t*)out, ldo);
  return hipGetLastError() == hipSuccess ? WSL_OK : dfail(WSL_E_LAUNCH, "swiglu: launch failed");
}

}  // extern "C"
