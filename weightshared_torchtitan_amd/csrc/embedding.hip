// Factorized token embedding for gfx950:  out[t, :] = E[ids[t], :] . P^T
//
// E [vocab, k] is the rank-k token table and P [hidden, k] the k -> hidden projection
// (nn.Linear(k, hidden).weight layout). The gather is fused into the GEMM's x-operand
// loads (row t of x is row ids[t] of E), so gathered rows never round-trip through
// HBM. The reference's unfactorized counterpart is nn.Embedding(vocab, dim)
// (torchtitan/models/llama3/model/model.py:561,
//  torchtitan/experiments/qwen3/model/model.py:350).
#include "wsl_common.h"

namespace wsl {

hipError_t launch_factorized_embedding(const int64_t* ids, int64_t n_ids, const void* emb,
                                       int64_t lde, int64_t vocab, int64_t k, const void* proj,
                                       int64_t ldp, int64_t hidden, void* out, int64_t ldo,
                                       hipStream_t stream) {
  LoraArgs p;
  p.x = emb; p.ldx = lde;
  p.w = proj; p.ldw = ldp; p.w_dtype = kBF16; p.w_scale = nullptr;
  p.a = nullptr; p.lda = 0; p.b = nullptr; p.ldb = 0;
  p.scale = 0.f;
  p.y = out; p.ldy = ldo;
  p.M = n_ids; p.N = hidden; p.K = k; p.r = 0;
  p.ws = nullptr; p.ws_bytes = 0;
  p.stream = stream;
  p.gather = ids; p.gather_rows = vocab;
  if (prefill_supported(p)) return launch_prefill(p);
  return launch_generic(p);
}

}  // namespace wsl
