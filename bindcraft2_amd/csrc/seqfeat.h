// The design sequence's features (the front of one design step): designed
// logits -> the features AlphaFold reads and the sequence profile, and the
// trunk inputs built from them (target_feat, msa_feat, aatype), forward and
// backward.  One thread per residue (20 amino acids).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bc2n {

constexpr int SEQ_A = 20;  // amino acids of the designed logits

// softmax_weight, one_hot_weight, temperature, logit_scale
struct SeqScalars {
  float sw = 1.f, ohw = 0.f, temp = 1.f, ls = 1.f;
};

// feat, prof [N][20] from logits [N][20]; flags bit 0 marks a designed
// residue (the others pass their logits through both outputs).  `bias` [20]
// may be null; `sc4` (device [4], in SeqScalars order) overrides `s` when set.
void seqfeat_fwd(hipStream_t st, const float* logits, const uint8_t* flags, const float* bias,
                 SeqScalars s, const float* sc4, float omitted_half, int N, float* feat,
                 float* prof);
void seqfeat_bwd(hipStream_t st, const float* logits, const uint8_t* flags, const float* bias,
                 SeqScalars s, const float* sc4, float omitted_half, int N, const float* d_feat,
                 const float* d_prof, float* d_logits);

// target_feat [N][21] (feat, then a zero column), msa_feat [1][N][49] (feat in
// channels 0..19, prof in 25..44, zeros elsewhere), aatype [N] = argmax(feat)
// (first maximum), as float.
void design_inputs_fwd(hipStream_t st, const float* feat, const float* prof, int N, float* tf,
                       float* mf, float* aatype);
// d feat = d target_feat[:, :20] + d msa_feat[0, :, 0:20]; d prof = d msa_feat[0, :, 25:45]
void design_inputs_bwd(hipStream_t st, const float* dtf, const float* dmf, int N, float* d_feat,
                       float* d_prof);

}  // namespace bc2n
