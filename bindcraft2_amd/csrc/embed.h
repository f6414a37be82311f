// Input embedder (multimer): the four input Linears on target_feat and
// msa_feat and the relative-position encoding, forward and backward.
#pragma once
#include "common.h"
#include "runtime.h"

namespace bc2n {

namespace embed {
constexpr int NAA = 21;       // target_feat, padded by one column (20 + 1)
constexpr int NMF = 49;       // msa_feat channels
constexpr int CM = 256;       // msa_channel
constexpr int CZ = 128;       // pair_channel
constexpr int MAX_REL = 32;   // max_relative_idx
constexpr int MAX_CHAIN = 2;  // max_relative_chain
constexpr int REL_BINS = 2 * MAX_REL + 2;                          // 66
constexpr int CHAIN_BINS = 2 * MAX_CHAIN + 2;                      // 6
constexpr int REL_TOT = REL_BINS + 1 + CHAIN_BINS;                 // 73
}  // namespace embed

struct EmbedW {
  const float *w1d = nullptr, *b1d = nullptr;    // preprocess_1d   [21][256], [256]
  const float *wmsa = nullptr, *bmsa = nullptr;  // preprocess_msa  [49][256], [256]
  const float *wl = nullptr, *bl = nullptr;      // left_single     [21][128], [128]
  const float *wr = nullptr, *br = nullptr;      // right_single    [21][128], [128]
  const float *wpos = nullptr, *bpos = nullptr;  // position_activations [73][128], [128]
  const float* wcat = nullptr;                   // [21][512]: preprocess_1d | left | right
};

// Weights under param/{preprocess_1d, preprocess_msa, left_single,
// right_single}/ and position_activations under param/ or
// param/evoformer/~_relative_encoding/.
EmbedW embed_weights(WeightStore& ws);

// tf [N][21], mf [S][N][49], ids [N] (f32, as the reference passes them),
// offset [N][N] int32 or null (then residue_index[i] - residue_index[j])
//   -> msa [S][N][256], pair [N][N][128]
void embed_fwd(hipStream_t st, const EmbedW& w, int N, int S, const float* tf, const float* mf,
               const float* residue_index, const float* asym_id, const float* entity_id,
               const float* sym_id, const int32_t* offset, float* msa, float* pair);
// dmsa [S][N][256], dpair [N][N][128], tf [N][21] -> dtf [N][21], dmf [S][N][49]
void embed_bwd(hipStream_t st, const EmbedW& w, int N, int S, const float* dmsa,
               const float* dpair, const float* tf, float* dtf, float* dmf);

}  // namespace bc2n
