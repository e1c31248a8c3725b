// C ABI of libwsl (declared in include/wsl_lora.h): argument validation, the one-time
// device check, and dispatch to the prefill / decode / generic kernels.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <atomic>
#include <cstring>
#include <mutex>

#include "../../include/wsl_decode.h"
#include "../../include/wsl_lora.h"
#include "wsl_common.h"

namespace wsl {
namespace {
// WSL_OPT_* values (include/wsl_lora.h), 0 = the library's own choice.
std::atomic<int64_t> g_options[WSL_OPT_COUNT];
}  // namespace

int64_t option(int id) {
  return (id > 0 && id < WSL_OPT_COUNT) ? g_options[id].load(std::memory_order_relaxed) : 0;
}
}  // namespace wsl

namespace {

thread_local char g_err[512] = {0};

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_err() { g_err[0] = 0; }

// Checks once per device that it is a gfx950 part (the kernels are built for it only).
int check_device() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(WSL_E_DEVICE, "hipGetDevice failed: %s", hipGetErrorString(e));
  static std::mutex mu;
  static int checked[64] = {0};  // 0 unknown, 1 ok, -1 bad
  if (dev < 0 || dev >= 64) return fail(WSL_E_DEVICE, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lk(mu);
  if (checked[dev] == 0) {
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return fail(WSL_E_DEVICE, "hipGetDeviceProperties failed: %s", hipGetErrorString(e));
    checked[dev] = (std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) ? 1 : -1;
    if (checked[dev] < 0) {
      return fail(WSL_E_DEVICE, "device %d is %s; libwsl is built for gfx950 only", dev, prop.gcnArchName);
    }
  }
  if (checked[dev] < 0) return fail(WSL_E_DEVICE, "device %d is not gfx950", dev);
  return WSL_OK;
}

// ---- scratch of the no-allocation entry point (wsl_lora_linear_fwd_noalloc) ----
// One array per GPU, held for the life of the process. In host code `scratch` is only a
// stand-in for the device symbol: its device address comes from hipGetSymbolAddress, once
// per device with that device current, and only that address is ever passed to kernels.
static __device__ __align__(256) unsigned char scratch[WSL_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {nullptr};

__global__ void __launch_bounds__(256) zero_fill_kernel(uint4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// The current device's scratch address, set up on the first call on that device: the
// symbol's address, then the whole array zero-filled by a kernel on `stream` (the decode
// path's launch counter must start at zero; stale words elsewhere are then zero, which no
// launch tag matches) and the stream synchronised, so later calls on any stream see it.
// That first call must not be under graph capture: a captured fill would replay, and
// resetting the launch counter on every replay would repeat launch tags.
int noalloc_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(WSL_E_DEVICE, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(WSL_E_DEVICE, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cap);
    if (e != hipSuccess) return fail(WSL_E_LAUNCH, "hipStreamIsCapturing failed: %s", hipGetErrorString(e));
    if (cap != hipStreamCaptureStatusNone)
      return fail(WSL_E_INVALID_ARG, "the first wsl_lora_linear_fwd_noalloc call on a device sets up its scratch "
                                     "and may not be captured; call it once outside graph capture first");
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(WSL_E_DEVICE, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    zero_fill_kernel<<<dim3(1024), dim3(256), 0, stream>>>(reinterpret_cast<uint4*>(ptr),
                                                           (size_t)WSL_NOALLOC_SCRATCH_BYTES / 16);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return fail(WSL_E_LAUNCH, "scratch zero-fill failed: %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return WSL_OK;
}

enum class Path { kNone, kPrefill, kDecode, kGeneric };

Path choose_path(const wsl::LoraArgs& p) {
  if (p.M == 0) return Path::kNone;
  if (p.M <= wsl::kDecodePlainMaxM && wsl::decode_supported(p)) return Path::kDecode;
  if (wsl::prefill_supported(p)) return Path::kPrefill;
  return Path::kGeneric;
}

// Workspace layout: kCounterBytes holding the decode path's launch counter, then two halves
// of equal size H (half_of): the decode path's launch-tagged hand-off words live in
// [kCounterBytes, kCounterBytes + H), the prefill and generic paths' plain scratch (bf16 T,
// fp32 split partials) in [kCounterBytes + H, kCounterBytes + 2H). Whatever shapes share a
// workspace, a value left by a prefill or generic call never sits where a decode launch
// looks for a tagged word, so it can never be taken for one.
size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
size_t half_of(size_t bytes) {
  return bytes <= wsl::kCounterBytes ? 0 : ((bytes - wsl::kCounterBytes) / 2) & ~(size_t)255;
}
// Bytes of a workspace whose halves each hold `data` bytes.
size_t layout_bytes(size_t data) { return wsl::kCounterBytes + 2 * align256(data); }

size_t decode_data(int64_t M, int64_t N, int64_t K, int64_t r, int w_dtype, int groups = 1) {
  const size_t t = groups > 1 ? wsl::decode_grouped_workspace_bytes(M, N, K, r, groups, w_dtype)
                              : wsl::decode_workspace_bytes(M, N, K, r, w_dtype);
  // plan offsets start after the counter prefix; a shape no decode plan covers needs none
  return t > wsl::kCounterBytes ? t - wsl::kCounterBytes : 0;
}
size_t generic_data(int64_t M, int64_t r) { return (size_t)(M * r * 2); }
size_t prefill_data(int64_t M, int64_t N, int64_t K, int64_t r, int w_dtype) {
  return wsl::prefill_workspace_bytes(M, N, K, r, w_dtype);
}

// Upper bound over the paths a problem of this size can take (the path also depends on
// pointer alignment, which the size query does not see).
size_t workspace_upper_bound(int64_t M, int64_t N, int64_t K, int64_t r, int w_dtype) {
  size_t b = generic_data(M, r);
  const size_t pf = prefill_data(M, N, K, r, w_dtype);
  if (pf > b) b = pf;
  if (M >= 1 && M <= wsl::kDecodePlainMaxM) {
    const size_t d = decode_data(M, N, K, r, w_dtype);
    if (d > b) b = d;
  }
  return layout_bytes(b);
}

// The storage type the kernels see and the fp8 activation terms of a public w_dtype code:
// WSL_DTYPE_FP8_E4M3_ACT8 is an fp8 W whose prefill product takes one activation term.
int32_t kernel_dtype(int32_t w_dtype, int* terms) {
  *terms = 2;
  if (w_dtype == WSL_DTYPE_FP8_E4M3_ACT8) {
    *terms = 1;
    return WSL_DTYPE_FP8_E4M3;
  }
  return w_dtype;
}

int validate_sizes(int64_t M, int64_t N, int64_t K, int64_t r, int32_t w_dtype) {
  if (M < 0) return fail(WSL_E_SHAPE, "M must be >= 0 (got %lld)", (long long)M);
  if (N < 1) return fail(WSL_E_SHAPE, "N must be >= 1 (got %lld)", (long long)N);
  if (K < 1) return fail(WSL_E_SHAPE, "K must be >= 1 (got %lld)", (long long)K);
  if (r < 0 || r > WSL_MAX_RANK)
    return fail(WSL_E_SHAPE, "rank r must be in [0, %d] (got %lld)", WSL_MAX_RANK, (long long)r);
  if (M > ((int64_t)1 << 31) || N > ((int64_t)1 << 31) || K > ((int64_t)1 << 31))
    return fail(WSL_E_SHAPE, "M, N, K must each be below 2^31");
  if (w_dtype != WSL_DTYPE_BF16 && w_dtype != WSL_DTYPE_FP8_E4M3)
    return fail(WSL_E_DTYPE, "unsupported w_dtype %d", (int)w_dtype);
  return WSL_OK;
}


// Argument checks shared by the single and grouped entry points (sizes, pointers,
// leading dimensions, element alignment). Touches no device.
int validate_call(const void* x, int64_t ldx, const void* w, int64_t ldw, int32_t w_dtype,
                  const float* w_scale, const void* a, int64_t lda, const void* b, int64_t ldb,
                  const void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int64_t r) {
  int rc = validate_sizes(M, N, K, r, w_dtype);
  if (rc != WSL_OK) return rc;
  if (M > 0 && x == nullptr) return fail(WSL_E_INVALID_ARG, "x must not be NULL");
  if (M > 0 && y == nullptr) return fail(WSL_E_INVALID_ARG, "y must not be NULL");
  if (w == nullptr && r == 0) return fail(WSL_E_INVALID_ARG, "w is NULL and r == 0: nothing to compute");
  if (r > 0 && (a == nullptr || b == nullptr)) return fail(WSL_E_INVALID_ARG, "r > 0 needs a and b");
  if (w != nullptr && w_dtype == WSL_DTYPE_FP8_E4M3 && w_scale == nullptr)
    return fail(WSL_E_INVALID_ARG, "fp8 w needs w_scale");
  if (w_dtype == WSL_DTYPE_BF16 && w_scale != nullptr)
    return fail(WSL_E_INVALID_ARG, "w_scale is only valid with an fp8 w");
  if (ldx < K) return fail(WSL_E_SHAPE, "ldx (%lld) < K (%lld)", (long long)ldx, (long long)K);
  if (w != nullptr && ldw < K) return fail(WSL_E_SHAPE, "ldw (%lld) < K (%lld)", (long long)ldw, (long long)K);
  if (r > 0 && lda < K) return fail(WSL_E_SHAPE, "lda (%lld) < K (%lld)", (long long)lda, (long long)K);
  if (r > 0 && ldb < r) return fail(WSL_E_SHAPE, "ldb (%lld) < r (%lld)", (long long)ldb, (long long)r);
  if (ldy < N) return fail(WSL_E_SHAPE, "ldy (%lld) < N (%lld)", (long long)ldy, (long long)N);
  if (((uintptr_t)x & 1) || ((uintptr_t)y & 1) || ((uintptr_t)a & 1) || ((uintptr_t)b & 1) ||
      ((uintptr_t)w_scale & 3) || (w_dtype == WSL_DTYPE_BF16 && ((uintptr_t)w & 1)))
    return fail(WSL_E_ALIGN, "pointers must be aligned to their element size");
  return WSL_OK;
}

// Group widths of a grouped call: 1..WSL_MAX_GROUPS groups, each at least one column;
// *N receives their sum.
int validate_groups(int32_t n_groups, const int64_t* group_n, int64_t* N) {
  if (n_groups < 1 || n_groups > WSL_MAX_GROUPS)
    return fail(WSL_E_SHAPE, "n_groups must be in [1, %d] (got %d)", WSL_MAX_GROUPS, (int)n_groups);
  if (group_n == nullptr) return fail(WSL_E_INVALID_ARG, "group_n must not be NULL");
  int64_t n = 0;
  for (int g = 0; g < n_groups; ++g) {
    if (group_n[g] < 1) return fail(WSL_E_SHAPE, "group %d has width %lld (must be >= 1)", g, (long long)group_n[g]);
    if (group_n[g] > ((int64_t)1 << 31)) return fail(WSL_E_SHAPE, "group widths must be below 2^31");
    n += group_n[g];
  }
  *N = n;
  return WSL_OK;
}

wsl::LoraArgs make_args(const void* x, int64_t ldx, const void* w, int64_t ldw, int32_t w_dtype,
                        const float* w_scale, const void* a, int64_t lda, const void* b, int64_t ldb,
                        float scale, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int64_t r,
                        void* stream) {
  wsl::LoraArgs p;
  p.x = x; p.ldx = ldx;
  p.w = w; p.ldw = ldw; p.w_dtype = w_dtype; p.w_scale = w_scale;
  p.a = a; p.lda = lda; p.b = b; p.ldb = ldb;
  p.scale = scale;
  p.y = y; p.ldy = ldy;
  p.M = M; p.N = N; p.K = K; p.r = r;
  p.ws = nullptr; p.ws_bytes = 0;
  p.stream = reinterpret_cast<hipStream_t>(stream);
  p.gather = nullptr; p.gather_rows = 0;
  return p;
}

// Path choice, workspace and device checks, and the launch of one validated call (a
// grouped call with p.groups > 1 only reaches here on the prefill path).
int run_call(wsl::LoraArgs p, void* workspace, size_t workspace_bytes) {
  const Path path = choose_path(p);
  if (path == Path::kNone) return WSL_OK;
  size_t need;
  switch (path) {
    case Path::kDecode: need = decode_data(p.M, p.N, p.K, p.r, p.w_dtype, p.groups); break;
    case Path::kPrefill: need = prefill_data(p.M, p.N, p.K, p.r * p.groups, p.w_dtype); break;
    default: need = generic_data(p.M, p.r); break;
  }
  const size_t half = half_of(workspace_bytes);
  if (workspace == nullptr || workspace_bytes < layout_bytes(need))
    return fail(WSL_E_WORKSPACE, "workspace of %zu bytes required (got %zu)", layout_bytes(need), workspace_bytes);
  if ((uintptr_t)workspace & 255)
    return fail(WSL_E_ALIGN, "workspace must be 256-byte aligned");
  const int rc = check_device();
  if (rc != WSL_OK) return rc;
  if (path == Path::kDecode) {  // plan offsets include the counter prefix
    p.ws = workspace;
    p.ws_bytes = wsl::kCounterBytes + half;
  } else {
    p.ws = reinterpret_cast<char*>(workspace) + wsl::kCounterBytes + half;
    p.ws_bytes = half;
    p.red_cnt = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(workspace) + wsl::kRedCntOff);
  }
  hipError_t e;
  switch (path) {
    case Path::kDecode: e = wsl::launch_decode(p); break;
    case Path::kPrefill: e = wsl::launch_prefill(p); break;
    default: e = wsl::launch_generic(p); break;
  }
  if (e != hipSuccess) return fail(WSL_E_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return WSL_OK;
}

// Whether a validated grouped call (p.groups, p.gend set) runs as one launch of its path;
// otherwise its groups run one by one.
bool grouped_one_launch(const wsl::LoraArgs& p) {
  if (p.groups == 1 || p.r == 0) return true;
  const Path path = choose_path(p);
  if (path == Path::kDecode) return wsl::decode_groups_supported(p);
  if (path != Path::kPrefill) return false;
  // The prefill path's medium-M split form must be taken (with the same split count) by the
  // grouped launch exactly when each group alone takes it, so the groups' outputs stay those
  // of the single calls bit for bit; otherwise the groups go one by one. A grouped launch
  // that takes the in-launch split-K form runs whole: its split count follows the launch's
  // tiles, so a group may sum K in another order than its single call (within the bar). That
  // form's 128 x 128 tiles compute their group's T, so its group ends must fall on multiples
  // of 128; where they do not, the groups go one by one (each may still take the form).
  const auto medium = [&](int64_t n, int64_t rt) {
    if (p.r <= 64 && wsl::red_splits(p.M, n, p.K, p.w_dtype, p.w != nullptr, false) > 0) return 0;
    return wsl::medium_splits(p.M, n, p.K, rt, p.w_dtype, p.w != nullptr, false);
  };
  const bool red_shape = p.r <= 64 && wsl::red_splits(p.M, p.N, p.K, p.w_dtype, p.w != nullptr, false) > 0;
  if (red_shape) return wsl::groups_fit_tiles(p, 128) && wsl::prefill_groups_supported(p);
  const int ms = medium(p.N, p.r * p.groups);
  for (int g = 0; g < p.groups; ++g) {
    const int64_t n = p.gend[g] - (g > 0 ? p.gend[g - 1] : 0);
    if (medium(n, p.r) != ms) return false;
  }
  return wsl::prefill_groups_supported(p);
}

// A grouped call after validation: one launch when the path's grid respects the group
// ends, else one launch per group in order on the same stream (the workspace is reused
// stream-ordered). With `shared_base` every group reads the same W (and w_scale) rows
// through p.wmap; otherwise group g's W rows follow the previous groups'.
int run_grouped(wsl::LoraArgs p, int n_groups, const int64_t* group_n, bool shared_base, void* workspace,
                size_t workspace_bytes) {
  p.groups = n_groups;
  int64_t end = 0;
  for (int g = 0; g < n_groups; ++g) p.gend[g] = (end += group_n[g]);
  if (n_groups == 1 || p.r == 0) {
    p.groups = 1;
    return run_call(p, workspace, workspace_bytes);
  }
  if (grouped_one_launch(p)) return run_call(p, workspace, workspace_bytes);
  const int64_t wbytes = (p.w_dtype == WSL_DTYPE_FP8_E4M3) ? 1 : 2;
  int64_t n0 = 0;
  for (int g = 0; g < n_groups; ++g) {
    wsl::LoraArgs q = p;
    q.groups = 1;
    q.N = group_n[g];
    if (!shared_base) {
      if (p.w != nullptr) q.w = reinterpret_cast<const char*>(p.w) + n0 * p.ldw * wbytes;
      if (p.w_scale != nullptr) q.w_scale = p.w_scale + n0;
    }
    q.a = reinterpret_cast<const uint16_t*>(p.a) + (int64_t)g * p.r * p.lda;
    q.b = reinterpret_cast<const uint16_t*>(p.b) + n0 * p.ldb;
    q.y = reinterpret_cast<uint16_t*>(p.y) + n0;
    const int rc = run_call(q, workspace, workspace_bytes);
    if (rc != WSL_OK) return rc;
    n0 += group_n[g];
  }
  return WSL_OK;
}

// The input gradient's problem in the linear's terms: x = gy [M, N], w = W [N, K], a = A,
// b = B, y = dx [M, K].
wsl::LoraArgs bwd_input_args(const void* gy, int64_t ldg, const void* w, int64_t ldw, int32_t w_dtype,
                             const float* w_scale, const void* a, int64_t lda, const void* b, int64_t ldb, float scale,
                             void* dx, int64_t lddx, int64_t M, int64_t N, int64_t K, int64_t r, void* stream) {
  return make_args(gy, ldg, w, ldw, w_dtype, w_scale, a, lda, b, ldb, scale, dx, lddx, M, N, K, r, stream);
}

}  // namespace

extern "C" {

int wsl_version(void) { return 101; }

int wsl_set_option(int32_t option, int64_t value) {
  clear_err();
  bool ok;
  switch (option) {
    case WSL_OPT_PREFILL_STRIPS:
    case WSL_OPT_PREFILL_MEDIUM: ok = value == 0 || value == -1; break;
    case WSL_OPT_DECODE_WIDE: ok = value >= -1 && value <= 1; break;
    case WSL_OPT_PREFILL_SPLIT: ok = value == 0 || value == -1 || (value >= 2 && value <= 16); break;
    case WSL_OPT_FP8_PREFILL: ok = value >= 0 && value <= 2; break;
    case WSL_OPT_DECODE_PASSES: ok = value >= -1 && value <= 1; break;
    case WSL_OPT_DECODE_SPIN_LIMIT: ok = value >= -1 && value <= ((int64_t)1 << 30); break;
    case WSL_OPT_DECODE_RES_SPLITS: ok = value == 0 || (value >= 2 && value <= 8); break;
    case WSL_OPT_PREFILL_SHARED_T: ok = value >= -1 && value <= 2; break;
    default: return fail(WSL_E_INVALID_ARG, "unknown option %d", (int)option);
  }
  if (!ok) return fail(WSL_E_INVALID_ARG, "value %lld out of range for option %d", (long long)value, (int)option);
  wsl::g_options[option].store(value, std::memory_order_relaxed);
  return WSL_OK;
}

int wsl_get_option(int32_t option, int64_t* value) {
  clear_err();
  if (value == nullptr) return fail(WSL_E_INVALID_ARG, "value must not be NULL");
  if (option < 1 || option >= WSL_OPT_COUNT) return fail(WSL_E_INVALID_ARG, "unknown option %d", (int)option);
  *value = wsl::option(option);
  return WSL_OK;
}

int wsl_lora_linear_plan(int64_t M, int64_t K, int64_t r, int32_t n_groups, const int64_t* group_n,
                         int32_t w_dtype_in, wsl_plan_info* out) {
  clear_err();
  if (out == nullptr) return fail(WSL_E_INVALID_ARG, "out must not be NULL");
  int terms;
  const int32_t w_dtype = kernel_dtype(w_dtype_in, &terms);
  int64_t N = 0;
  int rc = validate_groups(n_groups, group_n, &N);
  if (rc != WSL_OK) return rc;
  rc = validate_sizes(M, N, K, r, w_dtype);
  if (rc != WSL_OK) return rc;
  std::memset(out, 0, sizeof(*out));
  // dense, 256-byte aligned stand-ins for the operands (only their alignment is read)
  const void* al = reinterpret_cast<const void*>((uintptr_t)256);
  wsl::LoraArgs p = make_args(al, K, al, K, w_dtype, w_dtype == WSL_DTYPE_FP8_E4M3 ? reinterpret_cast<const float*>(al)
                                                                                    : nullptr,
                              al, K, al, r, 2.f, const_cast<void*>(al), N, M, N, K, r, nullptr);
  p.fp8_terms = terms;
  p.red_cnt = reinterpret_cast<unsigned*>(const_cast<void*>(al));
  p.ws = const_cast<void*>(al);  // a workspace of the size the size query reports
  p.ws_bytes = SIZE_MAX;
  p.groups = n_groups;
  int64_t end = 0;
  for (int g = 0; g < n_groups; ++g) p.gend[g] = (end += group_n[g]);
  if (n_groups == 1 || r == 0) p.groups = 1;
  if (choose_path(p) == Path::kNone) return WSL_OK;
  out->launches = 1;
  if (!grouped_one_launch(p)) {  // group by group: the first group's plan
    out->launches = n_groups;
    p.groups = 1;
    p.N = group_n[0];
  }
  out->strip_tiles = out->k_splits = 1;
  switch (choose_path(p)) {
    case Path::kDecode: out->path = WSL_PATH_DECODE; break;
    case Path::kGeneric: out->path = WSL_PATH_GENERIC; break;
    default: {
      const wsl::PrefillPlan pl = wsl::plan_prefill(p);
      out->path = pl.form;
      out->tile_m = pl.tile_m;
      out->tile_n = pl.tile_n;
      out->rank_blocks = pl.rank_blocks;
      out->rank_prepass = pl.prepass ? 1 : 0;
      out->shared_t = pl.shared_t ? 1 : 0;
      out->strip_tiles = pl.strips;
      out->k_splits = pl.splits;
      out->workgroups = (int32_t)pl.workgroups;
    }
  }
  return WSL_OK;
}

const char* wsl_last_error(void) { return g_err; }

int wsl_lora_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, int32_t w_dtype_in,
                                    size_t* bytes) {
  clear_err();
  int terms;
  const int32_t w_dtype = kernel_dtype(w_dtype_in, &terms);
  if (bytes == nullptr) return fail(WSL_E_INVALID_ARG, "bytes must not be NULL");
  int rc = validate_sizes(M, N, K, r, w_dtype);
  if (rc != WSL_OK) return rc;
  *bytes = workspace_upper_bound(M, N, K, r, w_dtype);
  return WSL_OK;
}

int wsl_lora_linear_fwd(const void* x, int64_t ldx, const void* w, int64_t ldw, int32_t w_dtype_in,
                        const float* w_scale, const void* a, int64_t lda, const void* b,
                        int64_t ldb, float scale, void* y, int64_t ldy, int64_t M, int64_t N,
                        int64_t K, int64_t r, void* workspace, size_t workspace_bytes,
                        void* stream) {
  clear_err();
  int terms;
  const int32_t w_dtype = kernel_dtype(w_dtype_in, &terms);
  const int rc = validate_call(x, ldx, w, ldw, w_dtype, w_scale, a, lda, b, ldb, y, ldy, M, N, K, r);
  if (rc != WSL_OK) return rc;
  wsl::LoraArgs p = make_args(x, ldx, w, ldw, w_dtype, w_scale, a, lda, b, ldb, scale, y, ldy, M, N, K, r, stream);
  p.fp8_terms = terms;
  return run_call(p, workspace, workspace_bytes);
}

int wsl_lora_linear_fwd_noalloc(const void* x, int64_t ldx, const void* w, int64_t ldw, int32_t w_dtype_in,
                                const float* w_scale, const void* a, int64_t lda, const void* b, int64_t ldb,
                                float scale, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int64_t r,
                                void* stream) {
  clear_err();
  int terms;
  const int32_t w_dtype = kernel_dtype(w_dtype_in, &terms);
  int rc = validate_call(x, ldx, w, ldw, w_dtype, w_scale, a, lda, b, ldb, y, ldy, M, N, K, r);
  if (rc != WSL_OK) return rc;
  wsl::LoraArgs p = make_args(x, ldx, w, ldw, w_dtype, w_scale, a, lda, b, ldb, scale, y, ldy, M, N, K, r,
                              stream);
  p.fp8_terms = terms;
  if (choose_path(p) == Path::kNone) return WSL_OK;
  // the exact need of the path this call takes (sizes and alignment are known here)
  size_t need;
  switch (choose_path(p)) {
    case Path::kDecode: need = layout_bytes(decode_data(M, N, K, r, w_dtype)); break;
    case Path::kPrefill: need = layout_bytes(prefill_data(M, N, K, r, w_dtype)); break;
    default: need = layout_bytes(generic_data(M, r)); break;
  }
  if (need > (size_t)WSL_NOALLOC_SCRATCH_BYTES)
    return fail(WSL_E_WORKSPACE, "this problem needs %zu bytes of scratch; the no-allocation entry point holds %zu "
                                 "(use wsl_lora_linear_fwd with a workspace)", need,
                (size_t)WSL_NOALLOC_SCRATCH_BYTES);
  rc = check_device();
  if (rc != WSL_OK) return rc;
  void* ws = nullptr;
  rc = noalloc_scratch(reinterpret_cast<hipStream_t>(stream), &ws);
  if (rc != WSL_OK) return rc;
  return run_call(p, ws, (size_t)WSL_NOALLOC_SCRATCH_BYTES);
}

int wsl_lora_linear_grouped_workspace_bytes(int64_t M, int64_t K, int64_t r, int32_t n_groups,
                                            const int64_t* group_n, int32_t w_dtype_in, size_t* bytes) {
  clear_err();
  int terms;
  const int32_t w_dtype = kernel_dtype(w_dtype_in, &terms);
  if (bytes == nullptr) return fail(WSL_E_INVALID_ARG, "bytes must not be NULL");
  int64_t N = 0;
  int rc = validate_groups(n_groups, group_n, &N);
  if (rc != WSL_OK) return rc;
  rc = validate_sizes(M, N, K, r, w_dtype);
  if (rc != WSL_OK) return rc;
  size_t b = layout_bytes(prefill_data(M, N, K, r * n_groups, w_dtype));
  if (M >= 1 && M <= wsl::kDecodePlainMaxM) {
    const size_t d = layout_bytes(decode_data(M, N, K, r, w_dtype, n_groups));
    if (d > b) b = d;
  }
  for (int g = 0; g < n_groups; ++g) {
    const size_t s1 = workspace_upper_bound(M, group_n[g], K, r, w_dtype);
    if (s1 > b) b = s1;
  }
  *bytes = b;
  return WSL_OK;
}

int wsl_lora_linear_grouped_fwd(const void* x, int64_t ldx, const void* w, int64_t ldw, int32_t w_dtype_in,
                                const float* w_scale, const void* a, int64_t lda, const void* b, int64_t ldb,
                                float scale, void* y, int64_t ldy, int64_t M, int64_t K, int64_t r,
                                int32_t n_groups, const int64_t* group_n, void* workspace,
                                size_t workspace_bytes, void* stream) {
  clear_err();
  int terms;
  const int32_t w_dtype = kernel_dtype(w_dtype_in, &terms);
  int64_t N = 0;
  int rc = validate_groups(n_groups, group_n, &N);
  if (rc != WSL_OK) return rc;
  rc = validate_call(x, ldx, w, ldw, w_dtype, w_scale, a, lda, b, ldb, y, ldy, M, N, K, r);
  if (rc != WSL_OK) return rc;
  wsl::LoraArgs p = make_args(x, ldx, w, ldw, w_dtype, w_scale, a, lda, b, ldb, scale, y, ldy, M, N, K, r, stream);
  p.fp8_terms = terms;
  return run_grouped(p, n_groups, group_n, false, workspace, workspace_bytes);
}

int wsl_lora_linear_bcast_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, int32_t n_groups,
                                          int32_t w_dtype, size_t* bytes) {
  if (n_groups < 1 || n_groups > WSL_MAX_GROUPS) {
    clear_err();
    return fail(WSL_E_SHAPE, "n_groups must be in [1, %d] (got %d)", WSL_MAX_GROUPS, (int)n_groups);
  }
  int64_t gn[WSL_MAX_GROUPS];
  for (int g = 0; g < n_groups; ++g) gn[g] = N;
  return wsl_lora_linear_grouped_workspace_bytes(M, K, r, n_groups, gn, w_dtype, bytes);
}

int wsl_lora_linear_bcast_fwd(const void* x, int64_t ldx, const void* w, int64_t ldw, int32_t w_dtype_in,
                              const float* w_scale, const void* a, int64_t lda, const void* b, int64_t ldb,
                              float scale, void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, int64_t r,
                              int64_t base_n, int64_t g, int32_t n_groups, void* workspace, size_t workspace_bytes,
                              void* stream) {
  clear_err();
  int terms;
  const int32_t w_dtype = kernel_dtype(w_dtype_in, &terms);
  if (n_groups < 1 || n_groups > WSL_MAX_GROUPS)
    return fail(WSL_E_SHAPE, "n_groups must be in [1, %d] (got %d)", WSL_MAX_GROUPS, (int)n_groups);
  if (w == nullptr) return fail(WSL_E_INVALID_ARG, "the shared-base form needs w");
  if (base_n < 1 || g < 1 || N < 1 || N % base_n != 0 || base_n % g != 0)
    return fail(WSL_E_SHAPE, "need N %% base_n == 0 and base_n %% g == 0 (N %lld, base_n %lld, g %lld)", (long long)N,
                (long long)base_n, (long long)g);
  const int64_t Nt = N * n_groups;
  int rc = validate_call(x, ldx, w, ldw, w_dtype, w_scale, a, lda, b, ldb, y, ldy, M, Nt, K, r);
  if (rc != WSL_OK) return rc;
  wsl::LoraArgs p = make_args(x, ldx, w, ldw, w_dtype, w_scale, a, lda, b, ldb, scale, y, ldy, M, Nt, K, r, stream);
  p.fp8_terms = terms;
  // column c of a group reads base row (c / (hpg D')) D' + c % D': the reference's
  // broadcast_add index map (D' = base_n / g templates' width, hpg = N / base_n heads each)
  const int64_t dw = base_n / g, hpg = N / base_n;
  p.wmap.P = (int)N;
  p.wmap.S = (int)(hpg * dw);
  p.wmap.D = (int)dw;
  p.wrows = base_n;
  int64_t gn[WSL_MAX_GROUPS];
  for (int q = 0; q < n_groups; ++q) gn[q] = N;
  return run_grouped(p, n_groups, gn, true, workspace, workspace_bytes);
}

int wsl_lora_linear_bwd_weights_supported(const void* x, int64_t ldx, const void* gy, int64_t ldg, const void* a,
                                          int64_t lda, const void* b, int64_t ldb, int64_t M, int64_t N, int64_t K,
                                          int64_t r) {
  const bool sizes_ok = validate_sizes(M, N, K, r, WSL_DTYPE_BF16) == WSL_OK && M >= 1;
  clear_err();  // a query leaves no error behind
  if (!sizes_ok) return 0;
  wsl::LoraArgs p = make_args(x, ldx, nullptr, 0, WSL_DTYPE_BF16, nullptr, a, lda, b, ldb, 1.f, nullptr, 0, M, N, K,
                              r, nullptr);
  return wsl::weight_grads_supported(p, gy, ldg) ? 1 : 0;
}

int wsl_lora_linear_bwd_weights_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, size_t* bytes) {
  clear_err();
  if (bytes == nullptr) return fail(WSL_E_INVALID_ARG, "bytes must not be NULL");
  const int rc = validate_sizes(M, N, K, r, WSL_DTYPE_BF16);
  if (rc != WSL_OK) return rc;
  *bytes = layout_bytes(M > 0 ? wsl::weight_grads_workspace_bytes(M, N, K, r, true, true) : 0);
  return WSL_OK;
}

int wsl_lora_linear_bwd_weights(const void* x, int64_t ldx, const void* gy, int64_t ldg, const void* a, int64_t lda,
                                const void* b, int64_t ldb, float scale, int64_t M, int64_t N, int64_t K, int64_t r,
                                void* dw, int64_t lddw, void* da, int64_t ldda, void* db, int64_t lddb,
                                void* workspace, size_t workspace_bytes, void* stream) {
  clear_err();
  int rc = validate_sizes(M, N, K, r, WSL_DTYPE_BF16);
  if (rc != WSL_OK) return rc;
  if (r == 0 && (da != nullptr || db != nullptr)) return fail(WSL_E_INVALID_ARG, "da and db need r > 0");
  if (M == 0 || (dw == nullptr && da == nullptr && db == nullptr)) return WSL_OK;
  if (x == nullptr || gy == nullptr) return fail(WSL_E_INVALID_ARG, "x and gy must not be NULL");
  if (r > 0 && (a == nullptr || b == nullptr)) return fail(WSL_E_INVALID_ARG, "r > 0 needs a and b");
  if (ldx < K) return fail(WSL_E_SHAPE, "ldx (%lld) < K (%lld)", (long long)ldx, (long long)K);
  if (ldg < N) return fail(WSL_E_SHAPE, "ldg (%lld) < N (%lld)", (long long)ldg, (long long)N);
  if (r > 0 && lda < K) return fail(WSL_E_SHAPE, "lda (%lld) < K (%lld)", (long long)lda, (long long)K);
  if (r > 0 && ldb < r) return fail(WSL_E_SHAPE, "ldb (%lld) < r (%lld)", (long long)ldb, (long long)r);
  if (dw != nullptr && lddw < K) return fail(WSL_E_SHAPE, "lddw (%lld) < K (%lld)", (long long)lddw, (long long)K);
  if (da != nullptr && ldda < K) return fail(WSL_E_SHAPE, "ldda (%lld) < K (%lld)", (long long)ldda, (long long)K);
  if (db != nullptr && lddb < r) return fail(WSL_E_SHAPE, "lddb (%lld) < r (%lld)", (long long)lddb, (long long)r);
  if (((uintptr_t)dw & 1) || ((uintptr_t)da & 1) || ((uintptr_t)db & 1) || ((uintptr_t)x & 1) ||
      ((uintptr_t)gy & 1) || ((uintptr_t)a & 1) || ((uintptr_t)b & 1))
    return fail(WSL_E_ALIGN, "pointers must be aligned to their element size");
  wsl::LoraArgs p = make_args(x, ldx, nullptr, 0, WSL_DTYPE_BF16, nullptr, a, lda, b, ldb, scale, nullptr, 0, M, N, K,
                              r, stream);
  const size_t need = wsl::weight_grads_workspace_bytes(M, N, K, r, true, true);
  if (workspace == nullptr || workspace_bytes < layout_bytes(need))
    return fail(WSL_E_WORKSPACE, "workspace of %zu bytes required (got %zu)", layout_bytes(need), workspace_bytes);
  if ((uintptr_t)workspace & 255) return fail(WSL_E_ALIGN, "workspace must be 256-byte aligned");
  rc = check_device();
  if (rc != WSL_OK) return rc;
  const size_t half = half_of(workspace_bytes);
  p.ws = reinterpret_cast<char*>(workspace) + wsl::kCounterBytes + half;
  p.ws_bytes = half;
  const hipError_t e = wsl::launch_weight_grads(p, gy, ldg, dw, lddw, da, ldda, db, lddb);
  if (e != hipSuccess) return fail(WSL_E_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return WSL_OK;
}

int wsl_lora_linear_bwd_input_supported(const void* gy, int64_t ldg, const void* w, int64_t ldw, int32_t w_dtype,
                                        const float* w_scale, const void* a, int64_t lda, const void* b, int64_t ldb,
                                        const void* dx, int64_t lddx, int64_t M, int64_t N, int64_t K, int64_t r) {
  int terms;
  const int32_t kdt = kernel_dtype(w_dtype, &terms);
  const bool sizes_ok = validate_sizes(M, N, K, r, kdt) == WSL_OK && M >= 1;
  clear_err();  // a query leaves no error behind
  if (!sizes_ok || gy == nullptr || w == nullptr || dx == nullptr || (r > 0 && (a == nullptr || b == nullptr)))
    return 0;
  if (kdt == WSL_DTYPE_FP8_E4M3 && w_scale == nullptr) return 0;
  const wsl::LoraArgs p = bwd_input_args(gy, ldg, w, ldw, kdt, w_scale, a, lda, b, ldb, 1.f, const_cast<void*>(dx),
                                         lddx, M, N, K, r, nullptr);
  return wsl::bwd_input_supported(p) ? 1 : 0;
}

int wsl_lora_linear_bwd_input_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t r, size_t* bytes) {
  clear_err();
  if (bytes == nullptr) return fail(WSL_E_INVALID_ARG, "bytes must not be NULL");
  const int rc = validate_sizes(M, N, K, r, WSL_DTYPE_BF16);
  if (rc != WSL_OK) return rc;
  *bytes = layout_bytes(M > 0 ? wsl::bwd_input_workspace_bytes(M, N, K, r) : 0);
  return WSL_OK;
}

int wsl_lora_linear_bwd_input(const void* gy, int64_t ldg, const void* w, int64_t ldw, int32_t w_dtype,
                              const float* w_scale, const void* a, int64_t lda, const void* b, int64_t ldb, float scale,
                              void* dx, int64_t lddx, int64_t M, int64_t N, int64_t K, int64_t r, void* workspace,
                              size_t workspace_bytes, void* stream) {
  clear_err();
  int terms;
  const int32_t kdt = kernel_dtype(w_dtype, &terms);
  int rc = validate_sizes(M, N, K, r, kdt);
  if (rc != WSL_OK) return rc;
  if (M == 0) return WSL_OK;
  if (gy == nullptr || w == nullptr || dx == nullptr) return fail(WSL_E_INVALID_ARG, "gy, w and dx must not be NULL");
  if (kdt == WSL_DTYPE_FP8_E4M3 && w_scale == nullptr)
    return fail(WSL_E_INVALID_ARG, "an fp8 w needs w_scale");
  if (r > 0 && (a == nullptr || b == nullptr)) return fail(WSL_E_INVALID_ARG, "r > 0 needs a and b");
  if (ldg < N) return fail(WSL_E_SHAPE, "ldg (%lld) < N (%lld)", (long long)ldg, (long long)N);
  if (ldw < K) return fail(WSL_E_SHAPE, "ldw (%lld) < K (%lld)", (long long)ldw, (long long)K);
  if (lddx < K) return fail(WSL_E_SHAPE, "lddx (%lld) < K (%lld)", (long long)lddx, (long long)K);
  if (r > 0 && lda < K) return fail(WSL_E_SHAPE, "lda (%lld) < K (%lld)", (long long)lda, (long long)K);
  if (r > 0 && ldb < r) return fail(WSL_E_SHAPE, "ldb (%lld) < r (%lld)", (long long)ldb, (long long)r);
  if (((uintptr_t)gy & 1) || ((uintptr_t)dx & 1) || ((uintptr_t)a & 1) || ((uintptr_t)b & 1) ||
      (kdt == WSL_DTYPE_BF16 && ((uintptr_t)w & 1)) || ((uintptr_t)w_scale & 3))
    return fail(WSL_E_ALIGN, "pointers must be aligned to their element size");
  wsl::LoraArgs p = bwd_input_args(gy, ldg, w, ldw, kdt, w_scale, a, lda, b, ldb, scale, dx, lddx, M, N, K, r, stream);
  if (!wsl::bwd_input_supported(p))
    return fail(WSL_E_SHAPE, "layout not taken (N %% 64, K %% 8 (16 for fp8), r %% 8, 16-byte aligned rows): "
                             "multiply by W^T");
  const size_t need = wsl::bwd_input_workspace_bytes(M, N, K, r);
  if (workspace == nullptr || workspace_bytes < layout_bytes(need))
    return fail(WSL_E_WORKSPACE, "workspace of %zu bytes required (got %zu)", layout_bytes(need), workspace_bytes);
  if ((uintptr_t)workspace & 255) return fail(WSL_E_ALIGN, "workspace must be 256-byte aligned");
  rc = check_device();
  if (rc != WSL_OK) return rc;
  const size_t half = half_of(workspace_bytes);
  p.ws = reinterpret_cast<char*>(workspace) + wsl::kCounterBytes + half;
  p.ws_bytes = half;
  p.red_cnt = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(workspace) + wsl::kRedCntOff);
  const hipError_t e = wsl::launch_bwd_input(p);
  if (e != hipSuccess) return fail(WSL_E_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return WSL_OK;
}

int wsl_lora_linear_fused_supported(int64_t M, int64_t N, int64_t K, int64_t r, int32_t fuse) {
  const bool sizes_ok = validate_sizes(M, N, K, r, WSL_DTYPE_BF16) == WSL_OK && M >= 1;
  clear_err();  // a query leaves no error behind
  if (!sizes_ok) return 0;
  // the sizes alone: every operand taken as 16-byte aligned with tight leading dimensions
  static char kAligned[16] __attribute__((aligned(16))) = {0};
  wsl::LoraArgs p;
  p.x = kAligned; p.ldx = K; p.w = kAligned; p.ldw = K; p.w_dtype = WSL_DTYPE_BF16; p.w_scale = nullptr;
  p.a = kAligned; p.lda = K; p.b = kAligned; p.ldb = r; p.scale = 1.f;
  p.y = kAligned; p.ldy = (fuse & WSL_FUSE_SWIGLU) ? N / 2 : N;
  p.M = M; p.N = N; p.K = K; p.r = r; p.ws = nullptr; p.ws_bytes = 0; p.stream = nullptr;
  p.gather = nullptr; p.gather_rows = 0;
  if (p.ldy % 4 != 0 || (r > 0 && r % 8 != 0)) return 0;
  const wsl::FusedArgs f{fuse, kAligned, 1e-6f, kAligned, N};
  return wsl::decode_fused_supported(p, f) ? 1 : 0;
}

int wsl_lora_linear_fused_fwd(const void* x, int64_t ldx, const void* norm_w, float eps, const void* w,
                              int64_t ldw, const void* a, int64_t lda, const void* b, int64_t ldb, float scale,
                              const void* residual, int64_t ldr, void* y, int64_t ldy, int64_t M, int64_t N,
                              int64_t K, int64_t r, int32_t fuse, void* workspace, size_t workspace_bytes,
                              void* stream) {
  clear_err();
  int rc = validate_sizes(M, N, K, r, WSL_DTYPE_BF16);
  if (rc != WSL_OK) return rc;
  if (fuse < 1 || fuse > 7 || ((fuse & WSL_FUSE_SWIGLU) && (fuse & WSL_FUSE_RESIDUAL)))
    return fail(WSL_E_INVALID_ARG, "fuse must combine WSL_FUSE_* flags (SWIGLU and RESIDUAL exclude each other)");
  if (M == 0) return WSL_OK;
  if (M > wsl::kDecodeMaxM) return fail(WSL_E_SHAPE, "the fused form is decode-shaped: M <= 64");
  if (x == nullptr || w == nullptr || y == nullptr) return fail(WSL_E_INVALID_ARG, "x, w and y must not be NULL");
  if (r > 0 && (a == nullptr || b == nullptr)) return fail(WSL_E_INVALID_ARG, "r > 0 needs a and b");
  if ((fuse & WSL_FUSE_RMSNORM) && norm_w == nullptr) return fail(WSL_E_INVALID_ARG, "norm_w must not be NULL");
  if ((fuse & WSL_FUSE_RESIDUAL) && residual == nullptr)
    return fail(WSL_E_INVALID_ARG, "residual must not be NULL");
  if (ldx < K || ldw < K || (r > 0 && (lda < K || ldb < r))) return fail(WSL_E_SHAPE, "leading dimension too small");
  if ((fuse & WSL_FUSE_SWIGLU) && N % 16 != 0) return fail(WSL_E_SHAPE, "SwiGLU needs N % 16 == 0 (interleaved rows)");
  const int64_t ny = (fuse & WSL_FUSE_SWIGLU) ? N / 2 : N;
  if (ldy < ny) return fail(WSL_E_SHAPE, "ldy too small");
  if ((fuse & WSL_FUSE_RESIDUAL) && ldr < N) return fail(WSL_E_SHAPE, "ldr < N");
  wsl::LoraArgs p;
  p.x = x; p.ldx = ldx; p.w = w; p.ldw = ldw; p.w_dtype = WSL_DTYPE_BF16; p.w_scale = nullptr;
  p.a = a; p.lda = lda; p.b = b; p.ldb = ldb; p.scale = scale; p.y = y; p.ldy = ldy;
  p.M = M; p.N = N; p.K = K; p.r = r; p.ws = workspace; p.ws_bytes = workspace_bytes;
  p.stream = reinterpret_cast<hipStream_t>(stream); p.gather = nullptr; p.gather_rows = 0;
  const wsl::FusedArgs f{fuse, norm_w, eps, residual, ldr};
  if (!wsl::decode_fused_supported(p, f))
    return fail(WSL_E_SHAPE, "the fused form does not cover this shape or alignment (wsl_lora_linear_fused_supported)");
  const size_t need = decode_data(M, N, K, r, WSL_DTYPE_BF16);
  if (workspace == nullptr || workspace_bytes < layout_bytes(need))
    return fail(WSL_E_WORKSPACE, "workspace of %zu bytes required (got %zu)", layout_bytes(need), workspace_bytes);
  if ((uintptr_t)workspace & 255) return fail(WSL_E_ALIGN, "workspace must be 256-byte aligned");
  rc = check_device();
  if (rc != WSL_OK) return rc;
  p.ws_bytes = wsl::kCounterBytes + half_of(workspace_bytes);
  const hipError_t e = wsl::launch_decode_fused(p, f);
  if (e != hipSuccess) return fail(WSL_E_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return WSL_OK;
}

}  // extern "C"

namespace {
// A chain's stages as launch arguments, after the checks that need no plan; the plan's own
// checks (shapes, alignment) follow in wsl::decode_chain_supported.
int chain_args(int64_t M, int32_t n, const wsl_chain_stage* st, wsl::LoraArgs* ps, wsl::FusedArgs* fs, int* after) {
  if (n < 1 || n > WSL_CHAIN_MAX_STAGES)
    return fail(WSL_E_SHAPE, "n_stages must be in [1, %d] (got %d)", WSL_CHAIN_MAX_STAGES, (int)n);
  if (st == nullptr) return fail(WSL_E_INVALID_ARG, "stages must not be NULL");
  if (M < 1 || M > 16) return fail(WSL_E_SHAPE, "chains take 1 <= M <= 16 (got %lld)", (long long)M);
  for (int s = 0; s < n; ++s) {
    const wsl_chain_stage& c = st[s];
    int rc = validate_sizes(M, c.N, c.K, c.r, WSL_DTYPE_BF16);
    if (rc != WSL_OK) return rc;
    const int fuse = c.fuse;
    if (fuse != 0 && fuse != WSL_FUSE_RMSNORM && fuse != (WSL_FUSE_RMSNORM | WSL_FUSE_SWIGLU) &&
        fuse != WSL_FUSE_RESIDUAL)
      return fail(WSL_E_INVALID_ARG, "stage %d: fuse must be 0, RMSNORM, RMSNORM|SWIGLU or RESIDUAL", s);
    if (c.x == nullptr || c.w == nullptr || c.y == nullptr)
      return fail(WSL_E_INVALID_ARG, "stage %d: x, w and y must not be NULL", s);
    if (c.r > 0 && (c.a == nullptr || c.b == nullptr)) return fail(WSL_E_INVALID_ARG, "stage %d: r > 0 needs a and b", s);
    if ((fuse & WSL_FUSE_RMSNORM) && c.norm_w == nullptr) return fail(WSL_E_INVALID_ARG, "stage %d: norm_w is NULL", s);
    if ((fuse & WSL_FUSE_RESIDUAL) && c.residual == nullptr)
      return fail(WSL_E_INVALID_ARG, "stage %d: residual is NULL", s);
    if (c.after_previous != 0 && c.after_previous != 1)
      return fail(WSL_E_INVALID_ARG, "stage %d: after_previous must be 0 or 1", s);
    const int g = c.n_groups;
    if (g < 1 || g > WSL_MAX_GROUPS || (fuse != 0 && g != 1))
      return fail(WSL_E_SHAPE, "stage %d: n_groups must be 1 with a fusion, 1..%d without", s, WSL_MAX_GROUPS);
    int64_t end = 0;
    wsl::LoraArgs p = make_args(c.x, c.ldx, c.w, c.ldw, WSL_DTYPE_BF16, nullptr, c.a, c.lda, c.b, c.ldb, c.scale,
                                c.y, c.ldy, M, c.N, c.K, c.r, nullptr);
    p.groups = g;
    for (int q = 0; q < g; ++q) {
      if (c.group_n[q] < 1) return fail(WSL_E_SHAPE, "stage %d: group %d has width %lld", s, q, (long long)c.group_n[q]);
      p.gend[q] = (end += c.group_n[q]);
    }
    if (g > 1 && end != c.N) return fail(WSL_E_SHAPE, "stage %d: the group widths sum to %lld, not N", s, (long long)end);
    const int64_t ny = (fuse & WSL_FUSE_SWIGLU) ? c.N / 2 : c.N;
    if (c.ldx < c.K || c.ldw < c.K || (c.r > 0 && (c.lda < c.K || c.ldb < c.r)) || c.ldy < ny ||
        ((fuse & WSL_FUSE_RESIDUAL) && c.ldr < c.N))
      return fail(WSL_E_SHAPE, "stage %d: leading dimension too small", s);
    ps[s] = p;
    fs[s] = wsl::FusedArgs{fuse, c.norm_w, c.eps, c.residual, c.ldr};
    after[s] = s > 0 ? c.after_previous : 0;
  }
  return WSL_OK;
}
}  // namespace

extern "C" {

int wsl_lora_linear_chain_supported(int64_t M, int32_t n_stages, const wsl_chain_stage* stages) {
  wsl::LoraArgs ps[WSL_CHAIN_MAX_STAGES];
  wsl::FusedArgs fs[WSL_CHAIN_MAX_STAGES];
  int after[WSL_CHAIN_MAX_STAGES];
  const bool ok = chain_args(M, n_stages, stages, ps, fs, after) == WSL_OK &&
                  wsl::decode_chain_supported(M, n_stages, ps, fs);
  clear_err();  // a query leaves no error behind
  return ok ? 1 : 0;
}

int wsl_lora_linear_chain_workspace_bytes(int64_t M, int32_t n_stages, const wsl_chain_stage* stages, size_t* bytes) {
  clear_err();
  if (bytes == nullptr) return fail(WSL_E_INVALID_ARG, "bytes must not be NULL");
  wsl::LoraArgs ps[WSL_CHAIN_MAX_STAGES];
  wsl::FusedArgs fs[WSL_CHAIN_MAX_STAGES];
  int after[WSL_CHAIN_MAX_STAGES];
  const int rc = chain_args(M, n_stages, stages, ps, fs, after);
  if (rc != WSL_OK) return rc;
  if (!wsl::decode_chain_supported(M, n_stages, ps, fs))
    return fail(WSL_E_SHAPE, "a stage's shape or alignment is not taken by chains (wsl_lora_linear_chain_supported)");
  *bytes = wsl::decode_chain_workspace_bytes(M, n_stages, ps, fs);
  return WSL_OK;
}

int wsl_lora_linear_chain_fwd(int64_t M, int32_t n_stages, const wsl_chain_stage* stages, void* workspace,
                              size_t workspace_bytes, void* stream) {
  clear_err();
  wsl::LoraArgs ps[WSL_CHAIN_MAX_STAGES];
  wsl::FusedArgs fs[WSL_CHAIN_MAX_STAGES];
  int after[WSL_CHAIN_MAX_STAGES];
  int rc = chain_args(M, n_stages, stages, ps, fs, after);
  if (rc != WSL_OK) return rc;
  if (!wsl::decode_chain_supported(M, n_stages, ps, fs))
    return fail(WSL_E_SHAPE, "a stage's shape or alignment is not taken by chains (wsl_lora_linear_chain_supported)");
  const size_t need = wsl::decode_chain_workspace_bytes(M, n_stages, ps, fs);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(WSL_E_WORKSPACE, "workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  if ((uintptr_t)workspace & 255) return fail(WSL_E_ALIGN, "workspace must be 256-byte aligned");
  rc = check_device();
  if (rc != WSL_OK) return rc;
  const hipError_t e = wsl::launch_decode_chain(M, n_stages, ps, fs, after, workspace,
                                                reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(WSL_E_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return WSL_OK;
}

int wsl_lora_linear_chain_status(void* workspace, void* stream, int32_t* failed) {
  clear_err();
  if (workspace == nullptr || failed == nullptr) return fail(WSL_E_INVALID_ARG, "workspace and failed must not be NULL");
  const int rc = check_device();
  if (rc != WSL_OK) return rc;
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  unsigned* word = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(workspace) + wsl::decode_chain_err_offset());
  unsigned v = 0;
  hipError_t e = hipMemcpyAsync(&v, word, sizeof(v), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e == hipSuccess && v != 0) {
    const unsigned zero = 0;
    e = hipMemcpyAsync(word, &zero, sizeof(zero), hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
  }
  if (e != hipSuccess) return fail(WSL_E_LAUNCH, "reading the chain status failed: %s", hipGetErrorString(e));
  *failed = v != 0 ? 1 : 0;
  return WSL_OK;
}

size_t wsl_tied_head_argmax_workspace_bytes(int64_t M) {
  return wsl::kCounterBytes + wsl::decode_argmax_keys_bytes(M);
}

int wsl_tied_head_argmax_supported(int64_t M, int64_t N, int64_t K) {
  const bool sizes_ok = validate_sizes(M, N, K, 0, WSL_DTYPE_BF16) == WSL_OK && M >= 1;
  clear_err();  // a query leaves no error behind
  if (!sizes_ok) return 0;
  static char kAligned[16] __attribute__((aligned(16))) = {0};
  wsl::LoraArgs p = make_args(kAligned, K, kAligned, K, WSL_DTYPE_BF16, nullptr, nullptr, 0, nullptr, 0, 0.f,
                              kAligned, N + (4 - N % 4) % 4, M, N, K, 0, nullptr);
  return wsl::decode_argmax_supported(p) ? 1 : 0;
}

int wsl_tied_head_argmax_fwd(const void* x, int64_t ldx, const void* w, int64_t ldw, int64_t N, int64_t K,
                             int64_t M, int64_t* out, void* workspace, size_t workspace_bytes, void* stream) {
  clear_err();
  int rc = validate_sizes(M, N, K, 0, WSL_DTYPE_BF16);
  if (rc != WSL_OK) return rc;
  if (M == 0) return WSL_OK;
  if (M > wsl::kDecodeMaxM) return fail(WSL_E_SHAPE, "the fused head is decode-shaped: M <= 64");
  if (N > ((int64_t)1 << 32) - 1) return fail(WSL_E_SHAPE, "N must be below 2^32 (indices live in 32 bits)");
  if (x == nullptr || w == nullptr || out == nullptr) return fail(WSL_E_INVALID_ARG, "x, w and out must not be NULL");
  if (ldx < K || ldw < K) return fail(WSL_E_SHAPE, "leading dimension too small");
  if (((uintptr_t)x & 1) || ((uintptr_t)w & 1) || ((uintptr_t)out & 7))
    return fail(WSL_E_ALIGN, "pointers must be aligned to their element size");
  // y is not written; the plan check takes out (8-byte aligned) as a stand-in of a y row
  wsl::LoraArgs p = make_args(x, ldx, w, ldw, WSL_DTYPE_BF16, nullptr, nullptr, 0, nullptr, 0, 0.f, out,
                              N + (4 - N % 4) % 4, M, N, K, 0, stream);
  if (!wsl::decode_argmax_supported(p))
    return fail(WSL_E_SHAPE, "the fused head does not cover this shape or alignment (wsl_tied_head_argmax_supported)");
  if (workspace == nullptr || workspace_bytes < wsl_tied_head_argmax_workspace_bytes(M))
    return fail(WSL_E_WORKSPACE, "workspace of %zu bytes required (got %zu)", wsl_tied_head_argmax_workspace_bytes(M),
                workspace_bytes);
  if ((uintptr_t)workspace & 255) return fail(WSL_E_ALIGN, "workspace must be 256-byte aligned");
  rc = check_device();
  if (rc != WSL_OK) return rc;
  p.ws = workspace;
  p.ws_bytes = wsl::kCounterBytes;
  const hipError_t e = wsl::launch_decode_argmax(p, reinterpret_cast<char*>(workspace) + wsl::kCounterBytes, out);
  if (e != hipSuccess) return fail(WSL_E_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return WSL_OK;
}

int wsl_factorized_embedding_fwd(const int64_t* ids, int64_t n_ids, const void* emb, int64_t lde,
                                 int64_t vocab, int64_t k, const void* proj, int64_t ldp,
                                 int64_t hidden, void* out, int64_t ldo, void* stream) {
  clear_err();
  if (n_ids < 0) return fail(WSL_E_SHAPE, "n_ids must be >= 0");
  if (vocab < 1 || k < 1 || hidden < 1) return fail(WSL_E_SHAPE, "vocab, k and hidden must be >= 1");
  if (k > 1024) return fail(WSL_E_SHAPE, "k must be <= 1024 (got %lld)", (long long)k);
  if (n_ids > ((int64_t)1 << 31) || hidden > ((int64_t)1 << 31) || vocab > ((int64_t)1 << 40))
    return fail(WSL_E_SHAPE, "sizes out of range");
  if (n_ids == 0) return WSL_OK;
  if (ids == nullptr || emb == nullptr || proj == nullptr || out == nullptr)
    return fail(WSL_E_INVALID_ARG, "ids, emb, proj and out must not be NULL");
  if (lde < k || ldp < k || ldo < hidden) return fail(WSL_E_SHAPE, "leading dimension too small");
  if (((uintptr_t)ids & 7) || ((uintptr_t)emb & 1) || ((uintptr_t)proj & 1) || ((uintptr_t)out & 1))
    return fail(WSL_E_ALIGN, "pointers must be aligned to their element size");
  int rc = check_device();
  if (rc != WSL_OK) return rc;
  hipError_t e = wsl::launch_factorized_embedding(ids, n_ids, emb, lde, vocab, k, proj, ldp, hidden,
                                                  out, ldo, reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(WSL_E_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return WSL_OK;
}

}  // extern "C"
