// Trunk modules: AF2 layers as sequences of gfx950 kernels.  Each module has
// a forward that writes `pair_out = pair_in + dropout(module(pair_in))` and
// fills a caller-owned save-set, and a backward that consumes the save-set
// and adds the module's input cotangent to the residual cotangent.  Scratch
// comes from the process arena; nothing is allocated inside a call once the
// arena has grown to the call's plan.
#pragma once
#include "runtime.h"
#include "kernels.h"

namespace bc2n {

// ---------------------------------------------------------- triangle attention
// modules.py TriangleAttention (+ Attention with pair bias and gating).
struct TriAttnW {
  int C = 0, H = 0, D = 0;
  const float *ln_g = nullptr, *ln_b = nullptr, *w2d = nullptr;  // w2d [C][H]
  const float* bqkvg = nullptr;  // [4HD]: zeros for q,k,v; gating_b for g
  const bf16* wqkvg_t = nullptr; // [4HD][C]
  const bf16* wqkvg = nullptr;   // [C][4HD]
  const bf16* wo_t = nullptr;    // [C][HD]
  const bf16* wo = nullptr;      // [HD][C]
  const float* bo = nullptr;     // [C]
};
TriAttnW triattn_weights(WeightStore& ws, const std::string& prefix);

size_t triattn_save_bytes(int N, int C, int H);
// per_column = "ending node" (the module runs on the transposed pair).
void triattn_fwd(hipStream_t st, const TriAttnW& w, bool per_column, int N,
                 const float* pair_in, const float* mask, const float* tbl,
                 float* pair_out, void* save);
void triattn_bwd(hipStream_t st, const TriAttnW& w, bool per_column, int N,
                 const float* pair_in, const float* mask, const float* tbl,
                 const void* save, const float* dout, float* din);

// ------------------------------------------------------ triangle multiplication
// modules.py:1044-1088 (fused projection weights).
struct TriMulW {
  int C = 0, I = 0;
  const float *ln_g = nullptr, *ln_b = nullptr, *cn_g = nullptr, *cn_b = nullptr;
  const float *bp = nullptr, *bg = nullptr, *bgl = nullptr, *bo = nullptr;
  const bf16* wcat = nullptr;    // [C][4I+C]  (GEMM column order)
  const bf16* wcat_t = nullptr;  // [4I+C][C]
  const bf16* wo = nullptr;      // [I][C]
  const bf16* wo_t = nullptr;    // [C][I]
};
TriMulW trimul_weights(WeightStore& ws, const std::string& prefix);
size_t trimul_save_bytes(int N, int C, int I);
void trimul_fwd(hipStream_t st, const TriMulW& w, bool outgoing, int N, const float* pair_in,
                const float* mask, const float* tbl, float* pair_out, void* save);
void trimul_bwd(hipStream_t st, const TriMulW& w, bool outgoing, int N, const float* pair_in,
                const float* mask, const float* tbl, const void* save, const float* dout,
                float* din);

}  // namespace bc2n
