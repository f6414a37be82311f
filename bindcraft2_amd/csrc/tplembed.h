// Template embedding around the template pair stack (one template, the
// eight constant feature projections hoisted into act_const).
#pragma once
#include "evoformer.h"

namespace bc2n {

struct TplEmbedW {
  const float *qn_g = nullptr, *qn_b = nullptr;  // query_embedding_norm
  const float *b8 = nullptr;                     // template_pair_embedding_8 bias
  const float *on_g = nullptr, *on_b = nullptr;  // output_layer_norm
  const float *bo = nullptr;                     // output_linear bias
  const h16 *w8 = nullptr, *w8_t = nullptr;     // [128][64] and its transpose
  const h16 *wo = nullptr, *wo_t = nullptr;     // [64][128] and its transpose
  StackW stack;
  int depth = 0;
};

// Weights under param/ (query_embedding_norm, template_pair_embedding_8,
// output_layer_norm, output_linear) and the stack's param/block{b}/...
TplEmbedW tplembed_weights(WeightStore& ws, int depth);
size_t tplembed_save_bytes(const TplEmbedW& w, int N);
// query [N][N][128], act_const [N][N][64] -> out [N][N][128]; key/enabled as
// for stack_fwd.  `out` is used as staging before it is written.
void tplembed_fwd(hipStream_t st, const TplEmbedW& w, int N, const float* query,
                  const float* act_const, const float* pmask, const uint32_t* key,
                  const uint32_t* enabled, bool dropout, float* out, void* save);
// dout [N][N][128] -> dquery [N][N][128] (act_const gets no gradient);
// `dquery` is used as staging before it is written.
void tplembed_bwd(hipStream_t st, const TplEmbedW& w, int N, const float* query,
                  const float* pmask, bool dropout, const void* save, const float* dout,
                  float* dquery);

}  // namespace bc2n
